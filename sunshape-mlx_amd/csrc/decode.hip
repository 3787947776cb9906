// Fused GQA decode/prefill attention over block-VQ key indices.
//
// One launch computes every query row of every (batch, KV head) group:
//   score[r][t] = sum_b LUT[r][b][idx[t][b]],  out[r] = softmax_t(score[r]) . V
// where LUT[r][b][c] = q'[r][b*8:(b+1)*8] . C[b][c] is built in LDS by every
// workgroup from the (scaled, rounded, permuted) query rows and the fp32
// codebook.  Semantics follow the reference's fused Metal kernels
// (kernels.py:142-223 and 303-378 for dense V, 588-687 and 772-860 for
// grouped V; per-head dispatch in attention.py:268-305), reorganised for
// CDNA4:
//   * grid.y = (batch, KV head, row group of R query rows): the R rows of one
//     GQA group share one pass over that head's indices and values, so K and
//     V are streamed once per KV head instead of once per query head;
//   * grid.x = split of the token axis ("flash-decoding"); each wave owns
//     64-token tiles: lane i gathers the 16 LUT entries of token i from LDS,
//     the tile's softmax is updated with wave reductions, and the value pass
//     maps 16-byte value loads to lanes (lanes-per-token = head_dim / dims-
//     per-lane);
//   * splits are merged by the last workgroup of each group to finish
//     (agent-scope release/acquire around one atomic counter), so a decode
//     step is a single kernel launch.
// Softmax runs in log2 units (LUT pre-multiplied by log2 e, exp2 on the
// hardware exp unit), accumulating in float32.
#include <atomic>
#include <mutex>
#include <type_traits>

#include "encode_wave.hpp"

namespace ss {

struct DecodeCommon {
    const void *q;
    const int32_t *perm;
    const float *centroids;
    const uint4 *codebook;       // split-fp16 codebook of the matrix-core LUT build (il8)
    const float *codebook_mul;   // its power-of-two scale (device memory)
    const uint8_t *idx;
    void *out;
    float *part_ml;   // [cols][splits][R] (m, l)
    float *part_acc;  // [cols][splits][R][D]
    int *part_cnt;    // [cols * cnt_stride] splits finished (in-kernel merge); zero between calls
    int cnt_stride;   // ints between two columns' counters (own cache lines: no contention)
    int fused_merge;  // MFMA kernel: merge the splits in-kernel (else a merge launch)
    int q_dtype, out_dtype;
    int n_q_heads, n_kv_heads, rep, n_rg;
    int64_t t_q, rows_total;
    int n_centroids;
    int64_t cap, t_kv;
    float scale;
    int causal;
    int64_t q_offset;
    int n_splits, tiles_per_split;
    // matrix-core kernel: tokens (a multiple of 8) every split but the last
    // takes beyond tiles_per_split * 64, so the last split, which then
    // ends at t_kv with that many fewer, has room for a fused step's work
    int split_pad = 0;
    // bounded waits of the matrix-core kernel: sleeps before a wait gives
    // up, and the sticky per-device word a give-up sets (kWait* bits)
    int spin_limit;
    unsigned int *wait_fail;
    // the same bits stored (not accumulated) into a word of pinned host
    // memory, which the host reads after the fact without synchronising
    unsigned int *wait_host;
    // fp16 heavy-block key dims of a mixed-precision codec (matrix-core
    // kernels of hybrid caches): [rows][nhd] halves of codec-basis dims
    // heavy_dims[0..nhd); nhd 0: none (every block scores from the LUT)
    const __half *kheavy;
    const int32_t *heavy_dims;
    int nhd;
    // matrix-core kernel writing the output itself (one split, or the
    // in-kernel merge): rows accumulated in a transformed basis leave as
    // y @ rot ([D][D] float32, row k = basis vector k); null: as they are
    const float *rot = nullptr;
};
constexpr int kMaxHeavyMfma = 32;  // heavy dims the matrix-core kernels take

// Bits of the wait-failure word: which bounded wait gave up.
constexpr unsigned kWaitBarrier = 1u;  // compute-wave barrier
constexpr unsigned kWaitSlot = 2u;     // loader: ring slot still held by its consumer
constexpr unsigned kWaitTile = 4u;     // compute wave: ring tile not yet published

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / kWave;
constexpr int kLutStride = 256;  // LUT entries reserved per (row, block)
constexpr int kBlockDim = 8;
constexpr int kMaxSplits = 512;  // split weights of the merge live in LDS

// Split-fp16 operands of the matrix-core LUT build: x = hi + lo / kSplitScale
// with hi = fp16(x), lo = fp16((x - hi) * kSplitScale).
constexpr float kSplitScale = 2048.f;
// The prepared codebook is scaled by 2^-e so that max |C| * 2^-e < 2^kCbMaxExp.
constexpr int kCbMaxExp = 14;

constexpr int pow2_ceil(int x) { return x <= 1 ? 1 : 2 * pow2_ceil((x + 1) / 2); }

// ---------------------------------------------------------------------------
// Value formats.  Each lane of a token group holds DPL consecutive dims.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void unpack16(const uint4 &u, float *x);

template <>
__device__ __forceinline__ void unpack16<__half>(const uint4 &u, float *x) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        __half2 h = *reinterpret_cast<const __half2 *>(&w[i]);
        float2 f = __half22float2(h);
        x[2 * i] = f.x;
        x[2 * i + 1] = f.y;
    }
}

template <>
__device__ __forceinline__ void unpack16<__hip_bfloat16>(const uint4 &u, float *x) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[2 * i] = __uint_as_float(w[i] << 16);
        x[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}

template <>
__device__ __forceinline__ void unpack16<float>(const uint4 &u, float *x) {
    x[0] = __uint_as_float(u.x);
    x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z);
    x[3] = __uint_as_float(u.w);
}

template <int D, typename T>
struct VDense {
    static constexpr int DPL = 16 / (int)sizeof(T);
    static constexpr int LPT = D / DPL;
    static constexpr int TPI = kWave / LPT;
    static constexpr int ITERS = kWave / TPI;
    struct Args {
        const T *v;
    };
    struct Raw {
        uint4 u;
    };
    __device__ static __forceinline__ Raw load(const Args &a, int64_t row, int lt, bool ok) {
        Raw r;
        r.u = ok ? *reinterpret_cast<const uint4 *>(a.v + row * D + lt * DPL)
                 : make_uint4(0u, 0u, 0u, 0u);
        return r;
    }
    __device__ static __forceinline__ void decode(const Args &, const Raw &r, int, float *x) {
        unpack16<T>(r.u, x);
    }
};

template <int D, int BITS, typename SZ>
struct VGrouped {
    static constexpr int VPW = 32 / BITS;
    static constexpr int NW = (D + VPW - 1) / VPW;
    static constexpr int DPL = VPW;
    static constexpr int LPT = pow2_ceil(NW);
    static constexpr int TPI = kWave / LPT;
    static constexpr int ITERS = kWave / TPI;
    static_assert(LPT <= kWave, "packed row too wide");
    struct Args {
        const uint32_t *packed;
        const SZ *scales;
        const SZ *zeros;
        int group;
        int n_groups;
    };
    struct Raw {
        uint32_t w;
        float s0, z0, s1, z1;
    };
    __device__ static __forceinline__ float ld(const SZ *p, int64_t i) {
        if constexpr (sizeof(SZ) == 4)
            return p[i];
        else
            return __half2float(p[i]);
    }
    __device__ static __forceinline__ Raw load(const Args &a, int64_t row, int lt, bool ok) {
        Raw r{0u, 0.f, 0.f, 0.f, 0.f};
        if (ok && lt < NW) {
            r.w = a.packed[row * NW + lt];
            const int d0 = lt * VPW;
            const int d1 = min(d0 + VPW - 1, D - 1);
            const int g0 = d0 / a.group, g1 = d1 / a.group;
            const int64_t sb = row * a.n_groups;
            r.s0 = ld(a.scales, sb + g0);
            r.z0 = ld(a.zeros, sb + g0);
            r.s1 = ld(a.scales, sb + g1);
            r.z1 = ld(a.zeros, sb + g1);
        }
        return r;
    }
    __device__ static __forceinline__ void decode(const Args &a, const Raw &r, int lt, float *x) {
        const int d0 = lt * VPW;
        const int g0 = d0 / a.group;
#pragma unroll
        for (int k = 0; k < VPW; ++k) {
            const float qv = (float)((r.w >> (k * BITS)) & ((1u << BITS) - 1u));
            const bool hi = ((d0 + k) / a.group) != g0;
            x[k] = fmaf(qv, hi ? r.s1 : r.s0, hi ? r.z1 : r.z0);
        }
    }
};

// TurboQuant values (reference value_codecs.py:136-177): per token a norm n
// and one BITS-bit Lloyd-Max code per dim of the rotated unit vector, packed
// like the grouped codes (kernels.py pack_indices).  A lane's dims decode to
// level[code] and the token's weight carries n, so the kernel accumulates
// p * n * level[code], the value in the rotated basis: since every token shares
// the rotation R, sum_t p_t (n_t C[idx_t] @ R) = (sum_t p_t n_t C[idx_t]) @ R,
// so the kernel accumulates in the rotated basis and R is applied once per
// output row: by the split-merge launch, or by rotate_rows_kernel when a
// single split writes the rows itself.
template <int D, int BITS>
struct VTurbo {
    static constexpr int VPW = 32 / BITS;
    static constexpr int NW = (D + VPW - 1) / VPW;
    static constexpr int DPL = VPW;
    static constexpr int LPT = pow2_ceil(NW);
    static constexpr int TPI = kWave / LPT;
    static constexpr int ITERS = kWave / TPI;
    static_assert(LPT <= kWave, "packed row too wide");
    struct Args {
        const uint32_t *packed;  // [rows][NW] words
        const float *norms;      // [rows]
        float lv[16];            // the 2^BITS levels, ascending (already x 1/sqrt(D))
        // keys of mixed-precision codecs: the heavy blocks' dims kept in
        // fp16 ([rows][nhd], codec basis), scored exactly beside the LUT
        const __half *kheavy;    // or null
        const int *heavy_dims;   // [nhd] codec-basis dims
        int nhd;                 // multiple of 8, <= kMaxHeavyDims
    };
    struct Raw {
        uint32_t w;
        float n;
    };
    __device__ static __forceinline__ Raw load(const Args &a, int64_t row, int lt, bool ok) {
        Raw r{0u, 0.f};
        if (ok && lt < NW) {
            r.w = a.packed[row * NW + lt];
            r.n = a.norms[row];
        }
        return r;
    }
    // level[code] by a select tree on the code bits (levels are uniform
    // kernel arguments; no indexed register access)
    __device__ static __forceinline__ float level(const Args &a, uint32_t code) {
        float v[1 << BITS];
#pragma unroll
        for (int i = 0; i < (1 << BITS); ++i) v[i] = a.lv[i];
#pragma unroll
        for (int b = 0; b < BITS; ++b) {
            const bool bit = (code >> b) & 1u;
#pragma unroll
            for (int i = 0; i < (1 << (BITS - 1 - b)); ++i) v[i] = bit ? v[2 * i + 1] : v[2 * i];
        }
        return v[0];
    }
    // Levels of every pair of adjacent codes, staged in LDS as float2: a
    // word decodes with one bit-field extract and one 8-byte LDS read per two
    // codes; the token's norm scales its softmax weight instead of each value.
    static constexpr int kPairs = 1 << (2 * BITS);
    // the pair table, then the heavy dims' query values
    static constexpr int kMaxHeavyDims = 64;
    static constexpr int kHeavyOffset = kPairs * 2;  // floats
    static constexpr int kLdsBytes = kPairs * 8 + 4 * kMaxHeavyDims * 4;
    static constexpr bool kHeavyKeys = true;
    static constexpr bool kTokenScale = true;
    static_assert(VPW % 2 == 0, "codes pair up within a word");
    __device__ static __forceinline__ void stage(float *lds, const Args &a, int, int tid, int nt) {
        float2 *t2 = reinterpret_cast<float2 *>(lds);
        for (int i = tid; i < kPairs; i += nt)
            t2[i] = make_float2(level(a, (uint32_t)i & ((1u << BITS) - 1u)),
                                level(a, (uint32_t)i >> BITS));
    }
    __device__ static __forceinline__ void decode_lds(const float *lds, const Args &, const Raw &r,
                                                      int, float *x) {
        const float2 *t2 = reinterpret_cast<const float2 *>(lds);
#pragma unroll
        for (int k = 0; k < VPW; k += 2) {
            const float2 v = t2[__builtin_amdgcn_ubfe(r.w, k * BITS, 2 * BITS)];
            x[k] = v.x;
            x[k + 1] = v.y;
        }
    }
    __device__ static __forceinline__ float token_scale(const Raw &r) { return r.n; }
};

// SunShape block-VQ values (value backend "sunshape", reference
// cache.py:614-623, 785-800): per token NBV = D / BD uint8 centroid indices
// of BD-dim blocks in the value codec's basis.  The value codebook is staged
// in LDS beside the key LUT in fp32 (64 KB per workgroup: at D = 128 two
// workgroups each take half the head dim and both compute the scores); an
// fp16 copy would move each centroid by up to 2^-12 of itself, which over a
// long cache of near-cancelling values reached 1e-3 of the output.  A lane
// takes 16 consecutive codec dims (16 / BD
// blocks, one 4- or 2-byte index group) and reads their centroids from LDS;
// accumulation runs in the codec basis and the transform back to the
// original basis (inverse permutation or rotation, as a D x D matrix) is
// applied per output row after the merge.
template <int D, int BD>
struct VSunV {
    // three waves per SIMD: the LDS gathers of one hide behind the others' FMAs
    static constexpr int kThreads = 768;
    // the codebook stays fp32 (the values the reference reads, exactly); a
    // head dim whose codebook passes 64 KB is split over two workgroups
    static constexpr int kSlabs = D * 256 * 4 > 65536 ? 2 : 1;
    static constexpr int DS = D / kSlabs;            // dims of one workgroup
    // the slab's fp32 centroids (256 per block), then the heavy dims' query values
    static constexpr int kMaxHeavyDims = 64;
    static constexpr int kHeavyOffset = DS * 256;  // floats
    static constexpr int kLdsBytes = DS * 256 * 4 + 4 * kMaxHeavyDims * 4;
    static constexpr bool kHeavyKeys = true;
    static constexpr int DPL = 16;
    static constexpr int BPL = DPL / BD;  // blocks per lane
    static constexpr int NBV = D / BD, NBVS = DS / BD;
    static constexpr int LPT = DS / DPL;
    static constexpr int TPI = kWave / LPT;
    static constexpr int ITERS = kWave / TPI;
    static_assert(BD == 4 || BD == 8, "value block_dim 4 or 8");
    struct Args {
        const uint8_t *idx;  // [rows][NBV]
        const float *cb;     // [NBV][n_centroids][BD], n_centroids <= 256
        int n_centroids;
        // keys of mixed-precision codecs: the heavy blocks' dims kept in
        // fp16 ([rows][nhd], codec basis), scored exactly beside the LUT
        const __half *kheavy;    // or null
        const int *heavy_dims;   // [nhd] codec-basis dims
        int nhd;                 // multiple of 8, <= kMaxHeavyDims
    };
    struct Raw {
        uint32_t w;
    };
    // lt: lane group over the whole head dim (slab * LPT + lane group)
    __device__ static __forceinline__ Raw load(const Args &a, int64_t row, int lt, bool ok) {
        Raw r{0u};
        if (ok) {
            const uint8_t *p = a.idx + row * NBV + lt * BPL;
            if constexpr (BPL == 4)
                r.w = *reinterpret_cast<const uint32_t *>(p);
            else
                r.w = *reinterpret_cast<const uint16_t *>(p);
        }
        return r;
    }
    // the slab's centroids -> lds [NBVS][256][BD] fp32 (entries past
    // n_centroids zero)
    __device__ static __forceinline__ void stage(float *lds, const Args &a, int slab, int tid,
                                                 int nt) {
        float4 *l4 = reinterpret_cast<float4 *>(lds);
        for (int i = tid; i < NBVS * 256 * BD / 4; i += nt) {
            const int f = i * 4, bl = f / (256 * BD), within = f - bl * (256 * BD);
            const int cc = within / BD;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (cc < a.n_centroids)
                v = *reinterpret_cast<const float4 *>(
                    a.cb + ((int64_t)(slab * NBVS + bl) * a.n_centroids + cc) * BD + within % BD);
            l4[i] = v;
        }
    }
    // lt: lane group within the slab
    __device__ static __forceinline__ void decode_lds(const float *lds, const Args &, const Raw &r,
                                                      int lt, float *x) {
        const float4 *l4 = reinterpret_cast<const float4 *>(lds);
#pragma unroll
        for (int i = 0; i < BPL; ++i) {
            const int bl = lt * BPL + i;
            const int cc = (int)((r.w >> (8 * i)) & 0xffu);
#pragma unroll
            for (int h = 0; h < BD / 4; ++h) {
                const float4 v = l4[((bl * 256 + cc) * BD) / 4 + h];
                x[i * BD + 4 * h + 0] = v.x;
                x[i * BD + 4 * h + 1] = v.y;
                x[i * BD + 4 * h + 2] = v.z;
                x[i * BD + 4 * h + 3] = v.w;
            }
        }
    }
};

// Dim slabs (workgroups sharing a split and column) and staged LDS bytes of a
// VALU value format: 1 and 0 unless the format declares kSlabs / kLdsBytes.
template <class VF, class = void>
struct VfSlabs {
    static constexpr int value = 1;
};
template <class VF>
struct VfSlabs<VF, std::void_t<decltype(VF::kSlabs)>> {
    static constexpr int value = VF::kSlabs;
};
template <class VF, class = void>
struct VfHeavy {  // the format's Args may carry fp16 heavy-block keys
    static constexpr bool value = false;
};
template <class VF>
struct VfHeavy<VF, std::void_t<decltype(VF::kHeavyKeys)>> {
    static constexpr bool value = VF::kHeavyKeys;
};
template <class VF, class = void>
struct VfHeavyMfma : std::false_type {};  // the matrix-core kernel scores fp16 heavy key dims
template <class VF>
struct VfHeavyMfma<VF, std::void_t<decltype(VF::kHeavyMfma)>> : std::integral_constant<bool, VF::kHeavyMfma> {};
template <class VF, class = void>
struct VfHeavyCapable : std::false_type {};  // the format has registers to spare for them
template <class VF>
struct VfHeavyCapable<VF, std::void_t<decltype(VF::kHeavyCapable)>>
    : std::integral_constant<bool, VF::kHeavyCapable> {};
// A matrix-core value format with the heavy-dim products compiled in: a
// separate kernel, launched only for calls that carry fp16 heavy key dims,
// so the plain kernels keep their registers and instruction schedule.
template <class VF>
struct WithHeavy : VF {
    static constexpr bool kHeavyMfma = true;
};
template <class T>
struct TypeTag {
    using type = T;
};
template <class VF, bool R>
struct RawUnitOf {  // a format's raw register unit (register-unit formats only)
    struct type {};
};
template <class VF>
struct RawUnitOf<VF, true> {
    using type = typename VF::Raw;
};
template <class VF, class = void>
struct VfRegUnits : std::false_type {};  // units loaded into registers, no LDS ring
template <class VF>
struct VfRegUnits<VF, std::void_t<decltype(VF::kRegUnits)>> : std::integral_constant<bool, VF::kRegUnits> {};
// How far (log2 units) the scores of a whole tile may rise above the running
// maxima before the matrix-core decodes reduce the maxima over the wave and
// rescale: the staged probabilities stay at most 2^lag, and most tiles after
// a split's first skip the reduction and the rescale.  Formats that stage
// them as bf16 hi/lo pairs take 8, the fp16 staging of the interleaved fp16
// values 4; without a kMaxLag a format takes 0 (every rise reduces).
template <class VF, class = void>
struct VfMaxLag {
    static constexpr float value = 0.f;
};
template <class VF>
struct VfMaxLag<VF, std::void_t<decltype(VF::kMaxLag)>> {
    static constexpr float value = VF::kMaxLag;
};

// The code words of a lane for one 64-token unit of token-interleaved codes
// ([cap / TPW][D] words per (batch, head)), straight from HBM into
// registers: per k-step, the NT words of dims NT*(lane%16) .. of the word
// block holding tokens 32ks + 8*(lane/16) ..; a lane whose tokens all lie
// past t_last reads the block holding t_last (its probabilities are 0).
// The words stay raw (the 2-bit shift is applied when the unit is used, so
// no instruction waits on the loads here).
template <int D, int NT, int TPW>
__device__ __forceinline__ void load_code_words(uint32_t (&cw)[2][NT], const uint32_t *codes, int64_t bh,
                                                int64_t cap, int64_t t0, int64_t t_last, int lane) {
    const int g = lane >> 4, l16 = lane & 15;
    const uint32_t *chead = codes + bh * (cap / TPW) * D;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
        const int64_t tk = min(t0 + 32 * ks + 8 * g, t_last);
        const uint32_t *src = chead + (tk / TPW) * D + (NT * l16) % D;
        const uint4 a = *reinterpret_cast<const uint4 *>(src);
        cw[ks][0] = a.x; cw[ks][1] = a.y; cw[ks][2] = a.z; cw[ks][3] = a.w;
        if constexpr (NT == 8) {
            const uint4 b = *reinterpret_cast<const uint4 *>(src + 4);
            cw[ks][4] = b.x; cw[ks][5] = b.y; cw[ks][6] = b.z; cw[ks][7] = b.w;
        }
    }
}
template <class VF, class = void>
struct VfArgsToLds : std::false_type {};  // the format's accumulator hand-off reads its Args
template <class VF>
struct VfArgsToLds<VF, std::void_t<decltype(&VF::to_lds_args)>> : std::true_type {};
template <class VF, class = void>
struct VfScaled {  // the format scales each token's weight (VF::token_scale)
    static constexpr bool value = false;
};
template <class VF>
struct VfScaled<VF, std::void_t<decltype(VF::kTokenScale)>> {
    static constexpr bool value = VF::kTokenScale;
};
template <class VF, class = void>
struct VfLds {
    static constexpr int value = 0;
};
template <class VF>
struct VfLds<VF, std::void_t<decltype(VF::kLdsBytes)>> {
    static constexpr int value = VF::kLdsBytes;
};

// ---------------------------------------------------------------------------
// Index rows: NB bytes per token (16 for head_dim 128, 8 for 64).
// ---------------------------------------------------------------------------
template <int NB>
struct IdxRow {
    uint32_t w[NB / 4];
    __device__ __forceinline__ void load(const uint8_t *p, bool ok) {
        if constexpr (NB == 16) {
            uint4 u = ok ? *reinterpret_cast<const uint4 *>(p) : make_uint4(0u, 0u, 0u, 0u);
            w[0] = u.x;
            w[1] = u.y;
            w[2] = u.z;
            w[3] = u.w;
        } else {
            static_assert(NB == 8, "unsupported block count");
            uint2 u = ok ? *reinterpret_cast<const uint2 *>(p) : make_uint2(0u, 0u);
            w[0] = u.x;
            w[1] = u.y;
        }
    }
    __device__ __forceinline__ uint32_t at(int b) const {
        return __builtin_amdgcn_ubfe(w[b >> 2], (b & 3) * 8, 8);
    }
};

template <class VF, class = void>
struct VfThreads {  // workgroup size of the VALU decode for this format
    static constexpr int value = kDecodeThreads;
};
template <class VF>
struct VfThreads<VF, std::void_t<decltype(VF::kThreads)>> {
    static constexpr int value = VF::kThreads;
};

template <int D, int R, int WAVES = kDecodeWaves>
constexpr size_t decode_lds_bytes() {
    return sizeof(float) * ((size_t)R * (D / kBlockDim) * kLutStride + (size_t)R * D +
                            (size_t)WAVES * kWave * R);
}

// The vector-ALU decode keeps a row's running maximum while a tile's scores
// stay at most kValuLag log2 units above it (fp32 probabilities up to
// 2^kValuLag).
constexpr float kValuLag = 8.f;

template <int D, int R, class VF>
__global__ void __launch_bounds__(VfThreads<VF>::value)
    decode_attn_kernel(DecodeCommon c, typename VF::Args va) {
    constexpr int TH = VfThreads<VF>::value, WV = TH / kWave;
    constexpr int NB = D / kBlockDim;
    constexpr int DPL = VF::DPL, LPT = VF::LPT, TPI = VF::TPI, ITERS = VF::ITERS;
    constexpr int CHUNK = ITERS < 16 ? ITERS : 16;
    static_assert(ITERS % CHUNK == 0, "chunking");
    static_assert(WV * R * (D + 2) <= R * NB * kLutStride, "merge scratch");
    // a format may split the head dim over SL workgroups (blockIdx.z) and
    // stage VLDS bytes of its own in LDS
    constexpr int SL = VfSlabs<VF>::value, DS = D / SL, VLDS = VfLds<VF>::value;
    static_assert(LPT * DPL >= DS, "value lanes cover the workgroup's dims");

    extern __shared__ __align__(16) float smem[];
    float *lut = smem;                          // [R][NB][kLutStride]
    float *qp = lut + R * NB * kLutStride;      // [R][D]
    float *pbuf = qp + R * D;                   // [waves][64][R]
    float *vlds = pbuf + WV * kWave * R;  // the format's staged data
    const int slab = SL > 1 ? (int)blockIdx.z : 0;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = tid >> 6;
    const int col = blockIdx.y;
    const int split = blockIdx.x;
    const int rg = col % c.n_rg;
    const int kvh = (col / c.n_rg) % c.n_kv_heads;
    const int64_t bb = col / (c.n_rg * c.n_kv_heads);
    const int64_t bh = bb * c.n_kv_heads + kvh;

    // Row r of this group: global row g = rg*R + r = rr*t_q + tq, query head
    // kvh*rep + rr (attention.py:220 reshape (B, Hkv, rep, Tq, D)).
    auto row_off = [&](int r) -> int64_t {
        const int64_t g = (int64_t)rg * R + r;
        const int64_t rr = g / c.t_q, tq = g - rr * c.t_q;
        return ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
    };
    auto row_ok = [&](int r) -> bool { return (int64_t)rg * R + r < c.rows_total; };

    // 1. query rows: round_to(q_dtype, q * scale) (attention.py:208), then
    //    the codec permutation (attention.py:228).
    for (int i = tid; i < R * D; i += TH) {
        const int r = i / D, j = i - r * D;
        float x = 0.f;
        if (row_ok(r)) {
            const int src = c.perm ? c.perm[j] : j;
            x = round_to(c.q_dtype, load_as_f32(c.q, c.q_dtype, row_off(r) + src) * c.scale);
        }
        qp[i] = x;
    }
    __syncthreads();

    // 2. LUT[r][b][c] = q'[r][b-block] . C[b][c] (kernels.py:178-190), in
    //    log2 units.  With fp16 heavy-block keys the blocks holding heavy
    //    dims are scored from those keys alone: their entries are 0.
    uint32_t heavy_blocks = 0;
    if constexpr (VfHeavy<VF>::value)
        if (va.kheavy)
            for (int j = 0; j < va.nhd; ++j)
                heavy_blocks |= 1u << (min(max(va.heavy_dims[j], 0), D - 1) / kBlockDim);
    const int nbc = NB * c.n_centroids;
    for (int e = tid; e < nbc; e += TH) {
        const int b = e / c.n_centroids, cc = e - b * c.n_centroids;
        const float4 *cp = reinterpret_cast<const float4 *>(c.centroids + (int64_t)e * kBlockDim);
        const float4 c0 = cp[0], c1 = cp[1];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float *qr = qp + r * D + b * kBlockDim;
            float dot = qr[0] * c0.x;
            dot = fmaf(qr[1], c0.y, dot);
            dot = fmaf(qr[2], c0.z, dot);
            dot = fmaf(qr[3], c0.w, dot);
            dot = fmaf(qr[4], c1.x, dot);
            dot = fmaf(qr[5], c1.y, dot);
            dot = fmaf(qr[6], c1.z, dot);
            dot = fmaf(qr[7], c1.w, dot);
            lut[(r * NB + b) * kLutStride + cc] = ((heavy_blocks >> b) & 1u) ? 0.f : dot * kLog2e;
        }
    }
    if constexpr (VLDS > 0) VF::stage(vlds, va, slab, tid, TH);
    if constexpr (VfHeavy<VF>::value) {
        // heavy dims' query values, in log2 units like the LUT
        float *qh = vlds + VF::kHeavyOffset;
        if (va.kheavy)
            for (int i = tid; i < R * va.nhd; i += TH) {
                const int r = i / va.nhd, j = i - r * va.nhd;
                qh[i] = qp[r * D + min(max(va.heavy_dims[j], 0), D - 1)] * kLog2e;
            }
    }
    __syncthreads();

    // 3. stream this split's tokens, 64 per wave-tile.
    const int64_t t_beg = (int64_t)split * c.tiles_per_split * kWave;
    const int64_t t_end = min(c.t_kv, t_beg + (int64_t)c.tiles_per_split * kWave);
    const int n_tiles = t_end > t_beg ? (int)((t_end - t_beg + kWave - 1) / kWave) : 0;
    const uint8_t *idx_head = c.idx + bh * c.cap * NB;
    const int64_t vrow0 = bh * c.cap;
    const int lt = lane % LPT, tg = lane / LPT;

    int64_t lim[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t g = (int64_t)rg * R + r;
        if (!row_ok(r))
            lim[r] = -1;
        else if (c.causal)
            lim[r] = c.q_offset + (g % c.t_q);
        else
            lim[r] = INT64_MAX;
    }

    float m[R], l[R], acc[R][DPL];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -1e30f;
        l[r] = 0.f;
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[r][k] = 0.f;
    }
    float *pw = pbuf + wv * kWave * R;

    for (int tile = wv; tile < n_tiles; tile += WV) {
        const int64_t t0 = t_beg + (int64_t)tile * kWave;
        typename VF::Raw vr[CHUNK];
#pragma unroll
        for (int j = 0; j < CHUNK; ++j) {
            const int64_t tv = t0 + j * TPI + tg;
            vr[j] = VF::load(va, vrow0 + tv, slab * LPT + lt, tv < t_end);
        }
        const int64_t tk = t0 + lane;
        const bool kok = tk < t_end;
        IdxRow<NB> ir;
        ir.load(idx_head + tk * NB, kok);

        float s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float *lr = lut + r * NB * kLutStride;
            float a = 0.f;
#pragma unroll
            for (int b = 0; b < NB; ++b) a += lr[b * kLutStride + ir.at(b)];
            s[r] = a;
        }
        if constexpr (VfHeavy<VF>::value) {
            if (va.kheavy) {  // uniform: exact dot products over the heavy dims
                const float *qh = vlds + VF::kHeavyOffset;
                const uint4 *kp = reinterpret_cast<const uint4 *>(va.kheavy + (vrow0 + tk) * va.nhd);
                float hs[R];
#pragma unroll
                for (int r = 0; r < R; ++r) hs[r] = 0.f;
                for (int j8 = 0; j8 < va.nhd / 8; ++j8) {
                    float kv[8];
                    unpack16<__half>(kok ? kp[j8] : make_uint4(0u, 0u, 0u, 0u), kv);
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int e = 0; e < 8; ++e)
                            hs[r] = fmaf(qh[r * va.nhd + j8 * 8 + e], kv[e], hs[r]);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) s[r] += hs[r];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) s[r] = (kok && tk <= lim[r]) ? s[r] : -INFINITY;
        // a tile whose scores stay at most kValuLag log2 units above the
        // running maxima keeps them (fp32 probabilities up to 2^kValuLag):
        // no wave-wide reduction and no rescale of the accumulators
        uint64_t above = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) above |= __builtin_amdgcn_ballot_w64(s[r] > m[r] + kValuLag);
        const bool moved = above != 0;
        float corr[R];
        if (moved) {
            float tmax[R];
            if constexpr (R == 4) {
                wave_max4_dpp(s, tmax);  // DPP lane moves, the four rows interleaved
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r) tmax[r] = wave_max(s[r]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float mn = fmaxf(m[r], tmax[r]);
                corr[r] = fast_exp2(m[r] - mn);
                const float p = fast_exp2(s[r] - mn);
                l[r] = fmaf(l[r], corr[r], p);
                m[r] = mn;
                s[r] = p;
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                corr[r] = 1.f;
                s[r] = fast_exp2(s[r] - m[r]);
                l[r] += s[r];
            }
        }
        if constexpr (R == 4) {
            *reinterpret_cast<float4 *>(pw + lane * 4) = make_float4(s[0], s[1], s[2], s[3]);
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) pw[lane * R + r] = s[r];
        }
        wave_lds_sync();
        if (moved) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int k = 0; k < DPL; ++k) acc[r][k] *= corr[r];
        }

#pragma unroll
        for (int ch = 0; ch < ITERS; ch += CHUNK) {
            if (ch > 0) {
#pragma unroll
                for (int j = 0; j < CHUNK; ++j) {
                    const int64_t tv = t0 + (ch + j) * TPI + tg;
                    vr[j] = VF::load(va, vrow0 + tv, slab * LPT + lt, tv < t_end);
                }
            }
#pragma unroll
            for (int j = 0; j < CHUNK; ++j) {
                const int tl = (ch + j) * TPI + tg;
                float pr[R];
                if constexpr (R == 4) {
                    const float4 p4 = *reinterpret_cast<const float4 *>(pw + tl * 4);
                    pr[0] = p4.x;
                    pr[1] = p4.y;
                    pr[2] = p4.z;
                    pr[3] = p4.w;
                } else {
#pragma unroll
                    for (int r = 0; r < R; ++r) pr[r] = pw[tl * R + r];
                }
                float x[DPL];
                if constexpr (VLDS > 0)
                    VF::decode_lds(vlds, va, vr[j], lt, x);
                else
                    VF::decode(va, vr[j], lt, x);
                if constexpr (VfScaled<VF>::value) {
                    const float ts = VF::token_scale(vr[j]);
#pragma unroll
                    for (int r = 0; r < R; ++r) pr[r] *= ts;
                }
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int k = 0; k < DPL; ++k) acc[r][k] = fmaf(pr[r], x[k], acc[r][k]);
            }
        }
        wave_lds_sync();
    }

    // 4. reduce the wave: token groups (lanes sharing lt), then l over lanes.
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int k = 0; k < DPL; ++k) {
            float v = acc[r][k];
#pragma unroll
            for (int o = LPT; o < kWave; o <<= 1) v += __shfl_xor(v, o);
            acc[r][k] = v;
        }
        l[r] = wave_sum(l[r]);
    }
    __syncthreads();  // every wave is done with the LUT; reuse it
    float *wm = smem;                        // [waves][R]
    float *wl = wm + WV * R;       // [waves][R]
    float *wa = wl + WV * R;       // [waves][R][DS]
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wm[wv * R + r] = m[r];
            wl[wv * R + r] = l[r];
        }
    }
    if (tg == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < DPL; ++k) {
                const int d = lt * DPL + k;
                if (d < DS) wa[(wv * R + r) * DS + d] = acc[r][k];
            }
    }
    __syncthreads();

    const int S = c.n_splits;
    for (int i = tid; i < R * DS; i += TH) {
        const int r = i / DS, d = i - r * DS, dd = slab * DS + d;
        float M = -1e30f;
#pragma unroll
        for (int w = 0; w < WV; ++w) M = fmaxf(M, wm[w * R + r]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < WV; ++w) {
            const float f = fast_exp2(wm[w * R + r] - M);
            L = fmaf(wl[w * R + r], f, L);
            A = fmaf(wa[(w * R + r) * DS + d], f, A);
        }
        if (S == 1) {
            if (row_ok(r)) store_from_f32(c.out, c.out_dtype, row_off(r) + dd, L > 0.f ? A / L : 0.f);
        } else {
            const int64_t slot = ((int64_t)col * S + split) * R + r;
            c.part_acc[slot * D + dd] = A;
            // every slab computes the same (M, L); slab 0 stores them
            if (dd == 0) *reinterpret_cast<float2 *>(c.part_ml + slot * 2) = make_float2(M, L);
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA decode for fp16 values stored 8-token interleaved: value element
// (token t, dim d) of a head lives at [t / 8][d][t % 8], so 16 bytes give a
// lane 8 consecutive tokens of one dim -- the K-major operand layout of
// v_mfma_f32_16x16x32_f16.  P.V runs on the matrix cores as
// O[row][dim] = sum_t P[row][t] V[t][dim] with M = query rows, K = tokens,
// N = dims.  P enters as an fp16 hi/lo pair (rows 0-3 hi, rows 4-7 lo) of
// p * 2^11, which keeps ~22 mantissa bits and stays in fp16's normal range;
// accumulation is fp32.  Four query rows (one GQA group) per workgroup.
//
// The workgroup is warp-specialised: NC compute waves and one loader wave.
// The loader streams the split's 64-token tiles (values and index rows) from
// HBM straight into an LDS ring with global_load_lds_dwordx4 -- no registers,
// no compute, so it can keep kDepth tiles in flight from the first cycle while
// the compute waves build the query x centroid LUT.  A wave that issues loads
// into a full memory pipeline stalls at the issue; only the loader ever does,
// so the compute waves never wait on anything but data that has landed.
// Tile j goes to slot j % kSlots and to compute wave j % NC.  Hand-off uses
// two LDS words per slot: ready[s] = j once tile j has landed (written by the
// loader after its vmcnt wait), done[s] = j once its consumer has copied the
// tile into registers.  Every wait on them is bounded (c.spin_limit sleeps,
// kSpinLimit by default): a wait that gives up sets its bit in the sticky
// per-device word c.wait_fail and the kernel ends normally with an invalid
// output, which ss_decode_wait_failures reports to the host.
// ---------------------------------------------------------------------------
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Probabilities staged for fp16 products as hi/lo pairs of p * kPScale: with
// a running-maximum lag of kPLag log2 units they reach 2^kPLag, and
// 2^kPLag * kPScale stays below the fp16 maximum; the lo parts stay normal
// down to p = 2^-14.
constexpr float kPScale = 2048.f;  // 2^11
constexpr float kPLag = 4.f;
constexpr int kMfmaRows = 4;
// Row stride (16-bit elements) of a wave's P staging: 64 tokens plus 8 of
// padding, so the 16 rows a matrix-core operand read touches start in
// different LDS banks.
constexpr int kPStride = 64 + 8;
static_assert((kPStride * 2) % 16 == 0, "16-byte P row reads");
constexpr int kLdsMax = 160 * 1024;  // LDS per workgroup on gfx950
constexpr int kSpinLimit = 1 << 20;  // bounded waits: ~0.03 s of s_sleep 1

template <class T>
using lds_t = __attribute__((address_space(3))) T;
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// Cache-policy bit sc1 of gfx940+ memory instructions: agent-coherent access
// (stores write through, loads do not hit a possibly stale line, of this
// XCD's L2).
constexpr int kCpolSc1 = 16;
// Cache-policy bit nt: streaming data, read once (the tile copies), so it
// does not displace what later steps reuse.
constexpr int kCpolNt = 2;

// Raw buffer resource over [p, p + bytes) (dword 3 of a raw gfx9 buffer
// descriptor); accesses past `bytes` read zero and drop writes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_buffer(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}

// LDS address of a shared-memory object as an address-space-3 pointer (the
// low 32 bits of a generic pointer into LDS are the LDS offset).
template <class T>
__device__ __forceinline__ lds_t<T> *to_lds(const void *p) {
    return reinterpret_cast<lds_t<T> *>(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

// s_waitcnt vmcnt(N), leaving the other counters unconstrained (gfx9 layout:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Wait until the oldest of k outstanding tiles (LPT loads each) has landed.
template <int LPT, int K>
__device__ __forceinline__ void wait_oldest_tile(int k) {
    if constexpr (K >= 1) {
        if (k >= K) {
            wait_vmcnt<(K - 1) * LPT>();
            return;
        }
        wait_oldest_tile<LPT, K - 1>(k);
    }
}

// Value formats that append a fused decode step's tokens (kStepShare).
template <class VF, class = void>
struct StepShareOf : std::false_type {};
template <class VF>
struct StepShareOf<VF, std::void_t<decltype(VF::kStepShare)>> : std::bool_constant<VF::kStepShare> {};
// Step formats whose step also attends a share of exact buffered tokens
// (VGilStep): the encoded tokens are the ones the buffer flushes.
template <class VF, class = void>
struct HybridStepOf : std::false_type {};
template <class VF>
struct HybridStepOf<VF, std::void_t<decltype(VF::kHybridStep)>> : std::bool_constant<VF::kHybridStep> {};
// Hybrid-step formats whose flushed values are quantised (VGilStep) rather
// than stored as fp16 (VIl8HybStep).
template <class VF, class = void>
struct StepQuantOf : std::false_type {};
template <class VF>
struct StepQuantOf<VF, std::void_t<decltype(VF::kStepQuant)>> : std::bool_constant<VF::kStepQuant> {};

template <int D, int NC, class VF>
struct WsCfg {
    static constexpr int kNB = D / kBlockDim;
    static constexpr int kSub = VF::kSub;         // 64-token sub-tiles per ring tile
    static constexpr int kTileV = VF::kTileV;     // value bytes of a ring tile
    static constexpr int kTileI1 = kWave * kNB;   // uint8 index rows of a sub-tile
    static constexpr int kTileI = kSub * kTileI1;
    static constexpr int kLoadsI = (kTileI + 1023) / 1024;
    static constexpr int kSlot = kTileV + kTileI;
    static constexpr int kLut = kNB * kLutStride * 16;  // float4 per (block, centroid)
    static constexpr int kPst = NC * VF::kPRows * kPStride * 2;  // P staging, 16-bit [rows][kPStride] per wave
    static constexpr int kFlagWords = 16;
    // ready[slot], done[slot][sub], barrier counter
    static constexpr int kFlags = (kFlagWords * (1 + kSub) + 4) * 4;
    // the split's share of a hybrid cache's token buffer: its query copy,
    // then its (m[R], l[R], acc[R][D]) partial
    static constexpr int kBufPart = VF::kHybridBuffer ? (2 * kMfmaRows + kMfmaRows * D) * 4 : 0;
    // a fused step's new index rows (4 tokens x NB bytes, 64 reserved) and
    // its encode's per-wave candidates (NC x 4 blocks x 4 tokens x 16 B)
    static constexpr int kStepLds = StepShareOf<VF>::value ? 64 + NC * 16 * 16 : 0;
    // a hybrid split's share of up to kShareLdsTok 16-bit buffered tokens,
    // keys then values [tok][D], copied in the prologue: on the private-ring
    // shapes (their ring has a fixed size, so the copy costs no ring slot)
    static constexpr int kShareFree = kLdsMax - (kLut + kPst + kFlags + kBufPart + kStepLds) -
                                      NC * 2 * kSlot;  // beside a private ring of 2 slots a wave
    static constexpr int kShareFit = kShareFree > 0 ? kShareFree / (4 * D) / 8 * 8 : 0;
    static constexpr int kShareLdsTok = (VF::kHybridBuffer &&
                                         (!StepShareOf<VF>::value || HybridStepOf<VF>::value) &&
                                         VF::kPrivateRing) ? (kShareFit < 32 ? kShareFit : 32) : 0;
    static constexpr int kShareLds = kShareLdsTok * D * 2 * 2;
    static constexpr int kRing = kLut + kPst + kFlags + kBufPart + kStepLds + kShareLds;
    static constexpr int kSlotsFit = (kLdsMax - kRing) / kSlot;
    static constexpr int kSlots = kSlotsFit < VF::kMaxSlots ? kSlotsFit : VF::kMaxSlots;
    static constexpr int kLoadsPerTile = VF::kLoadsV + kLoadsI;
    static_assert(kLoadsPerTile <= 63, "one ring tile within the vmcnt range");
    static constexpr int kDepthVm = 63 / kLoadsPerTile + 1;
    // one slot more than the tiles in flight, so a refill never waits on the
    // slowest consumer of the tile it replaces
    static constexpr int kDepth = kSlots - 1 < kDepthVm ? kSlots - 1 : kDepthVm;
    // wave-private rings (VF::kPrivateRing): no loader wave; every compute
    // wave copies its own 64-token units, kPrivSlots of them at a time
    static constexpr bool kPriv = VF::kPrivateRing;
    static constexpr int kPrivSlots = 2;
    static constexpr int kWaves = kPriv ? NC : NC + 1;
    static constexpr int kRingBytes = kPriv ? NC * kPrivSlots * kSlot : kSlots * kSlot;
    static constexpr int kLds = kRing + kRingBytes;
    static_assert(kSlots >= 2 && kSlots <= kFlagWords, "ring slots");
    static_assert(kTileV % 16 == 0, "16-byte tile sections");
    static_assert(kLds <= kLdsMax, "LDS budget");
    static_assert(!kPriv || kSub == 1, "private rings hold single 64-token units");
    static_assert(NC * kMfmaRows * (2 * D + 2) * 4 <= kRingBytes, "merge scratch");
    static_assert(2 * kMfmaRows * D * 4 <= kPst, "query staging");
    // LUT build on the matrix cores: tiles of 4 blocks x 16 centroids, each
    // compute wave owns kLutTiles of them, all in one 4-block group
    static constexpr int kLutTiles = (kNB / 4) * (kLutStride / 16) / NC;
    static_assert(kNB % 4 == 0 && (kNB / 4) * (kLutStride / 16) % NC == 0 &&
                      (kLutStride / 16) % kLutTiles == 0, "LUT split");
};

// Zero the fp16 values of tokens >= n_ok (0..8) in an 8-token group.
__device__ __forceinline__ uint4 mask_tokens(uint4 u, int n_ok) {
    uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = (2 * i) < n_ok ? 0x0000ffffu : 0u;
        const uint32_t hi = (2 * i + 1) < n_ok ? 0xffff0000u : 0u;
        w[i] &= (lo | hi);
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Value formats of the matrix-core decode kernel.  A format supplies the value
// bytes of a 64-token tile and their copies into the LDS ring (the loader),
// its tile data in registers (each compute lane holds token `lane` for P and
// the B operands of P.V), the P.V step for a tile given this lane's
// probabilities, and the hand-off of the accumulators to the workgroup
// combine as (hi, lo) parts per row and dim.  Accumulator lane layout (every
// format): acc[n] of lane l holds MFMA rows 4*(l/16) .. +3 of dims 16n + l%16.

// fp16 values, 8-token interleaved: element (t, d) at [t/8][d][t%8].  P is
// staged as fp16 hi/lo rows of p * 2^11 (A rows 0-3 hi, 4-7 lo, 8-15 zero)
// and P.V is v_mfma_f32_16x16x32_f16.
template <int D, int SUB = 1>
struct VIl8 {
    struct Args {
        const __half *v8;
    };
    static constexpr int NT = D / 16;
    static constexpr int kSub = SUB;
    static constexpr bool kHybridBuffer = false;  // fp16 caches have no token buffer
    // probabilities staged as fp16 hi/lo pairs of p * kPScale
    static constexpr float kMaxLag = kPLag;
    static constexpr bool kPrivateRing = false;   // 17 KB units: one loader wave, shared ring
    static constexpr int kTileV1 = kWave * D * 2;  // one 64-token sub-tile
    static constexpr int kTileV = kSub * kTileV1;
    static constexpr int kLoadsV = kTileV / 1024;
    static constexpr int kPRows = 8;
    static constexpr int kMaxSlots = 8;
    static constexpr int kComputeWaves = 4;  // one per SIMD: 272-byte tokens keep them busy
    struct Tile {
        uint4 v[2][NT];
    };
    struct State {};
    // values of tokens t0 .. t0 + 64*kSub - 1 (contiguous); in a tile that
    // reaches past the split's last token, 8-token blocks past it are
    // clamped to its block, so every copy stays in bounds
    template <class A>
    __device__ static void issue(const A &a, int64_t bh, int64_t cap, int64_t t0, int64_t t_last,
                                 uint32_t sb, int lane) {
        const char *vhead = reinterpret_cast<const char *>(a.v8 + bh * cap * D);
        const int64_t b0 = t0 / 8, blk_last = t_last / 8;
        if (t0 + kSub * kWave - 1 <= t_last) {  // uniform base + lane offset
            const char *base = vhead + b0 * D * 16;
#pragma unroll
            for (int i = 0; i < kLoadsV; ++i)
                __builtin_amdgcn_global_load_lds(base + (uint32_t)(i * 1024 + lane * 16),
                                                 reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                                 kCpolNt);
            return;
        }
#pragma unroll
        for (int i = 0; i < kLoadsV; ++i) {
            const int q = i * kWave + lane;  // 16-byte chunk of the tile
            const int64_t blk = min(b0 + q / D, blk_last);
            __builtin_amdgcn_global_load_lds(vhead + (blk * D + q % D) * 16,
                                             reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                             kCpolNt);
        }
    }
    __device__ static void copy(Tile &tv, const char *sb, int sub, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        sb += sub * kTileV1;
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
            for (int n = 0; n < NT; ++n)
                tv.v[s2][n] = *reinterpret_cast<const uint4 *>(sb + ((4 * s2 + g) * D + 16 * n + l16) * 16);
    }
    __device__ static void init(State &) {}
    __device__ static void pv(Tile &tv, State &, f32x4 (&acc)[NT], const float (&p)[kMfmaRows],
                              const float (&corr)[kMfmaRows], bool rescale, int n_in, _Float16 *pw,
                              int lane) {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int r = 0; r < kMfmaRows; ++r) {
            const float x = p[r] * kPScale;
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            pw[r * kPStride + lane] = hi;
            pw[(r + 4) * kPStride + lane] = lo;
        }
        wave_lds_sync();
        // rescale only when some row's running max moved (wave-uniform;
        // after the first tiles it rarely does)
        if (rescale) {
            const f32x4 cv4 = f32x4{corr[0], corr[1], corr[2], corr[3]};
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= cv4;
        }
        if (n_in < kWave) {  // last, partial tile: zero tokens >= t_end
#pragma unroll
            for (int s2 = 0; s2 < 2; ++s2) {
                const int n_ok = min(max(n_in - 8 * (4 * s2 + g), 0), 8);
#pragma unroll
                for (int n = 0; n < NT; ++n) tv.v[s2][n] = mask_tokens(tv.v[s2][n], n_ok);
            }
        }
        const bool a_live = l16 < 8;  // A rows 0-3: hi parts, 4-7: lo parts, 8-15: zero
        // v_mfma_f32_16x16x32_f16 (full fp16 rate): K slots 8g .. 8g+7 of
        // lane l are tokens 32 s2 + 8g .. +7 in A (its P row) and in B (its
        // 8 tokens of one dim)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            f16x8 a = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
            if (a_live) a = *reinterpret_cast<const f16x8 *>(pw + l16 * kPStride + 32 * s2 + 8 * g);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const f16x8 bop = __builtin_bit_cast(f16x8, tv.v[s2][n]);
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop, acc[n], 0, 0, 0);
            }
        }
        wave_lds_sync();
    }
    // lanes 0-15 hold rows 0-3 (hi parts) of dims 16n + l16, lanes 16-31 the
    // lo parts: wa[hl][r][d] = acc / kPScale
    __device__ static void to_lds(const f32x4 (&acc)[NT], const State &, float *wa, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        if (g < 2) {
#pragma unroll
            for (int r = 0; r < kMfmaRows; ++r)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    wa[(g * kMfmaRows + r) * D + 16 * n + l16] = acc[n][r] * (1.f / kPScale);
        }
    }
};

// VIl8 over a hybrid cache: the same compressed tiles, and the recent-token
// buffer (keys and values in the original basis, buf_dtype elements at
// b*buf_sb + h*buf_sh + t*buf_st (+ dim)) attended as positions t_kv ..
// t_kv + t_buf - 1 in the same softmax.
template <int D>
struct VIl8Hyb : VIl8<D> {
    struct Args {
        const __half *v8;
        const void *kbuf, *vbuf;
        int buf_dtype;
        int64_t buf_sb, buf_sh, buf_st, t_buf;
    };
    static constexpr bool kHybridBuffer = true;
    static constexpr bool kHeavyCapable = true;
};

// VIl8 for one decode step that also appends its tokens: the cache holds
// t_kv tokens and the step's n_new newest (keys and values at
// kbuf / vbuf [b*buf_sb + h*buf_sh + j*buf_st + dim], t_buf = n_new) arrive
// with the call.  The last split encodes their keys exactly (the float32
// centroids, as the encoder), scores them from the LUT by their indices, as
// the cache's own tokens, and attends them with its tiles (the buffer-share
// partial of VIl8Hyb); the last split of row group 0 of each (batch, KV
// head) also writes their index rows and fp16 values into the cache at
// positions t_kv .. t_kv + n_new - 1, which the next call reads.
template <int D>
struct VIl8Step : VIl8<D> {
    struct Args {
        const __half *v8;
        const void *kbuf, *vbuf;
        int buf_dtype;
        int64_t buf_sb, buf_sh, buf_st, t_buf;
        const float *centroids;  // [n_blocks][n_centroids][8] float32
        const float *cb_norms;   // |C|^2 per prepared codebook lane (ss_codebook_f16x2)
        uint8_t *idx_out;        // the index cache the kernel reads (c.idx)
        __half *v8_out;          // the value cache (v8)
    };
    static constexpr bool kHybridBuffer = true;
    static constexpr bool kStepShare = true;
    static constexpr bool kHeavyCapable = false;
};
constexpr int kMaxStepTokens = 4;  // new tokens of one fused decode step (A rows 4s + r)

// VIl8Hyb for one decode step of a hybrid cache with fp16 values that also
// moves its tokens (the VGilStep protocol, below): the flushed tokens' fp16
// values are attended as they are and stored into the interleaved values
// (v8_out) at positions t_kv .., beside their index rows.
template <int D>
struct VIl8HybStep : VIl8<D> {
    struct Args : VIl8Hyb<D>::Args {
        const void *knew, *vnew;  // float16 [b*new_sb + h*new_sh + j*new_st + dim]
        int64_t new_sb, new_sh, new_st, n_rem, n_flush;
        const float *centroids;  // [n_blocks][n_centroids][8] float32
        const float *cb_norms;   // |C|^2 per prepared codebook lane (ss_codebook_f16x2)
        uint8_t *idx_out;        // the index cache the kernel reads (c.idx)
        __half *v8_out;          // the value cache (v8)
        void *kput, *vput;       // the buffer stores at the window (kbuf / vbuf)
    };
    static constexpr bool kHybridBuffer = true;
    static constexpr bool kStepShare = true;
    static constexpr bool kHybridStep = true;
    static constexpr bool kStepQuant = false;
    static constexpr bool kHeavyCapable = false;
};
// cache tokens the last split of a fused step hands to the other splits
// (about the time of its encode and share)
constexpr int64_t kStepShareTokens = 192;
// the same for a hybrid cache's fused step (VGilStep): its last split also
// waits, before its LUT barrier, for the flushed tokens' rows, cold in HBM
// (about 5 us at B=8, T=32K); measured there, the step took 43.6 / 42.4 /
// 41.1 / 40.2 us with 192 / 512 / 1024 / 1536 tokens handed over, and no
// less with more
constexpr int64_t kHybridStepShareTokens = 1536;
// Register-unit splits: rounds of units that wave 0 hands to the other waves
// when it first attends a share of buffered tokens (its copy waits behind
// the start-up traffic), and the rounds added when it also scores a hybrid
// step's flushed tokens
constexpr int kShareSkipRounds = 6;
constexpr int kStepSkipRounds = 3;


// Round two floats to bf16 (nearest even), packed: a in bits 0-15, b in 16-31.
__device__ __forceinline__ uint32_t bf16x2_rn(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}

// A 32-bit value the compiler cannot see as a literal, so the bitwise
// and-or of the code expansion below becomes a single v_and_or_b32 on
// registers (gfx9 three-operand forms take no literal operands).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t x) {
    uint32_t r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "i"(x));
    return r;
}

// Grouped asymmetric values (bits 2 or 4, NG = 1 or 2 groups per row, scale
// and zero of type SZT): v = code * s + z.  Codes are token-interleaved: per
// (b, h), u32 word (blk, d) of [cap / TPW][D] holds dim d of tokens blk*TPW ..
// +TPW-1, token i at bit BITS*(i/2) + 16*(i%2) (even tokens in the low half,
// odd ones in the high half), so two neighbouring tokens' codes of one dim
// sit in the two bf16 halves of a dword after one shift; scales/zeros are
// [cap][NG].  P.V = sum_t (p_t s_t) code_t + sum_t p_t z_t.  The first sum
// runs on the matrix cores (v_mfma_f32_16x16x32_bf16): A rows are w = p * s
// of each (group, row) split into bf16 hi/lo (rows 8g+0..3 hi, 8g+4..7 lo of
// group g), B the codes of 8 tokens of one dim as bf16 128 + code (bit
// pattern 0x4300 | code, exact), so the products carry 128 * sum_t w_t; the
// same A times an all-128 B (one more product per k-step) accumulates that
// term exactly alike, and the two are subtracted at the end.  The second sum
// accumulates per (row, group) in fp32 on the lanes.  N-tile n, column c
// holds dim 8c + n, so a lane reads its eight dims' words as two 16-byte
// LDS loads per k-step.
template <int D, int BITS, int NG, class SZT>
struct VGil {
    struct Args {
        const uint32_t *codes;
        const SZT *scales, *zeros;
        // recent-token buffer of a hybrid cache: keys and values in the
        // original basis, buf_dtype elements at b*buf_sb + h*buf_sh +
        // t*buf_st (+ dim), attended as positions t_kv .. t_kv + t_buf - 1
        // after the compressed tokens (t_buf = 0: none)
        const void *kbuf, *vbuf;
        int buf_dtype;
        int64_t buf_sb, buf_sh, buf_st, t_buf;
    };
    static constexpr int NT = D / 16;
    static constexpr int TPW = 32 / BITS;                 // tokens per code word
    static constexpr int kCodeBytes1 = kWave * D * BITS / 8;  // codes of a 64-token sub-tile
    static constexpr int kSzBytes1 = kWave * NG * (int)sizeof(SZT);
    // every compute wave copies its own 64-token units (3.5 KB at 2-bit)
    // into two private LDS slots: no loader wave and no hand-off flags.
    // Measured as a bare stream over the config-4 buffers, 8 waves x 2 units
    // in flight reach 6.3 TB/s (a single loader wave with 64-token tiles
    // reached 3.7 TB/s, with 256-token tiles 5.9 TB/s), and the compute
    // waves no longer wait on flags in a congested LDS.
    // (4-bit codes at D = 128, 5.5 KB units, do not fit 16 private slots
    // beside the LUT: they keep the loader wave and 128-token ring tiles)
    static constexpr bool kPrivateRing = kCodeBytes1 <= 2048;
    static constexpr int kSub = kPrivateRing ? 1 : (8192 / kCodeBytes1 < 4 ? 8192 / kCodeBytes1 : 4);
    static constexpr int kCodeBytes = kSub * kCodeBytes1;
    static constexpr int kSzBytes = kSub * kSzBytes1;
    static constexpr bool kHybridBuffer = true;  // hybrid caches: recent tokens join the pass
    // fp16 heavy key dims: on the private-ring shapes (the loader-wave shape
    // has no registers to spare for them)
    static constexpr bool kHeavyCapable = kPrivateRing;
    static constexpr int kSzLoads = (kSzBytes + 1023) / 1024;
    static constexpr int kTileV = kCodeBytes + 2 * kSzBytes;
    static constexpr int kLoadsV = kCodeBytes / 1024 + 2 * kSzLoads;
    static constexpr int kPRows = 16;
    static constexpr int kMaxSlots = 16;
    // two compute waves per SIMD: a 64-token step is a long chain of LDS
    // round trips (index rows, LUT gathers, P staging) that a second wave
    // overlaps (measured 5 % faster than one wave per SIMD at config 4)
    static constexpr int kComputeWaves = 8;
    static constexpr int kGroup = D / NG;
    static constexpr uint32_t kCodeMask = BITS == 2 ? 0x00030003u : 0x000f000fu;
    static constexpr uint32_t kBias = 0x43004300u;  // two bf16 128.0
    static_assert(BITS == 2 || BITS == 4, "bits");
    static_assert(NG == 1 || NG == 2, "groups per row");
    static_assert(NT == 8 || NT == 4, "n-tiles");
    static_assert(kSub >= 1 && kCodeBytes1 % 1024 == 0 && kSzBytes1 % 16 == 0, "tile sections");
    struct Tile {
        // per k-step, the lane's 8 tokens (32ks + 8*(lane/16) ..) of dims
        // 8*(lane%16) + n: their code word, shifted so that dword j of the
        // operand is ((cw >> BITS*j) & kCodeMask) | kBias
        uint32_t cw[2][NT];
        float s[NG], z[NG];  // scale / zero of token `lane`
    };
    // register units (private-ring shapes): a unit is loaded from HBM into
    // registers one unit ahead of its use, with no LDS copy
    static constexpr bool kRegUnits = kPrivateRing;
    static constexpr float kMaxLag = 8.f;  // bf16 hi/lo probabilities
    struct Raw {
        uint32_t cw[2][NT];  // unshifted words
        SZT s[NG], z[NG];
    };
    __device__ static void load(Raw &u, const Args &a, int64_t bh, int64_t cap, int64_t t0, int64_t t_last,
                                int lane) {
        load_code_words<D, NT, TPW>(u.cw, a.codes, bh, cap, t0, t_last, lane);
        const int64_t tok = min(t0 + lane, t_last);
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            u.s[k] = a.scales[(bh * cap + tok) * NG + k];
            u.z[k] = a.zeros[(bh * cap + tok) * NG + k];
        }
    }
    __device__ static void from_raw(Tile &tv, const Raw &u, int lane) {
        const int sh = BITS == 2 ? 8 * ((lane >> 4) & 1) : 0;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int n = 0; n < NT; ++n) tv.cw[ks][n] = u.cw[ks][n] >> sh;
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            tv.s[k] = (float)u.s[k];
            tv.z[k] = (float)u.z[k];
        }
    }
    struct State {
        f32x4 bias;               // 128 * sum of the staged A rows, laid out as acc
        float zs[kMfmaRows][NG];  // sum of p * z
    };
    __device__ static void issue(const Args &a, int64_t bh, int64_t cap, int64_t t0, int64_t t_last,
                                 uint32_t sb, int lane) {
        const char *chead = reinterpret_cast<const char *>(a.codes + bh * (cap / TPW) * D);
        const char *sp = reinterpret_cast<const char *>(a.scales + (bh * cap + t0) * NG);
        const char *zp = reinterpret_cast<const char *>(a.zeros + (bh * cap + t0) * NG);
        const int64_t wb0 = t0 / TPW;
        if (t0 + kSub * kWave - 1 <= t_last) {  // uniform bases + lane offsets
            const char *cb = chead + wb0 * D * 4;
#pragma unroll
            for (int i = 0; i < kCodeBytes / 1024; ++i)
                __builtin_amdgcn_global_load_lds(cb + (uint32_t)(i * 1024 + lane * 16),
                                                 reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                                 kCpolNt);
#pragma unroll
            for (int i = 0; i < kSzLoads; ++i) {
                const uint32_t off = (uint32_t)(i * 1024 + lane * 16);
                if (kSzBytes % 1024 == 0 || off < (uint32_t)kSzBytes) {
                    __builtin_amdgcn_global_load_lds(
                        sp + off, reinterpret_cast<lds_t<void> *>(sb + kCodeBytes + i * 1024), 16, 0,
                        kCpolNt);
                    __builtin_amdgcn_global_load_lds(
                        zp + off, reinterpret_cast<lds_t<void> *>(sb + kCodeBytes + kSzBytes + i * 1024),
                        16, 0, kCpolNt);
                }
            }
            return;
        }
        // a tile reaching past the split's last token: code chunks (4 words
        // of one block) past its block clamp to that block, scale/zero
        // chunks past the one holding it clamp to that chunk
        const int64_t blk_last = t_last / TPW;
#pragma unroll
        for (int i = 0; i < kCodeBytes / 1024; ++i) {
            const int w = (i * kWave + lane) * 4;  // first word of the chunk
            const int64_t blk = min(wb0 + w / D, blk_last);
            __builtin_amdgcn_global_load_lds(chead + (blk * D + w % D) * 4,
                                             reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                             kCpolNt);
        }
        constexpr int kTokPerChunk = 16 / (NG * (int)sizeof(SZT));
        const int64_t ch_last = (t_last - t0) / kTokPerChunk;
#pragma unroll
        for (int i = 0; i < kSzLoads; ++i) {
            const int c = i * kWave + lane;
            if (kSzBytes % 1024 == 0 || c * 16 < kSzBytes) {
                const int64_t ch = min((int64_t)c, ch_last);
                __builtin_amdgcn_global_load_lds(
                    sp + ch * 16, reinterpret_cast<lds_t<void> *>(sb + kCodeBytes + i * 1024), 16, 0,
                    kCpolNt);
                __builtin_amdgcn_global_load_lds(
                    zp + ch * 16, reinterpret_cast<lds_t<void> *>(sb + kCodeBytes + kSzBytes + i * 1024),
                    16, 0, kCpolNt);
            }
        }
    }
    __device__ static void copy(Tile &tv, const char *sb, int sub, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        const char *cb = sb + sub * kCodeBytes1;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int tk = 32 * ks + 8 * g;  // first of the lane's 8 tokens
            const uint32_t *src = reinterpret_cast<const uint32_t *>(cb) + (tk / TPW) * D + (NT * l16) % D;
            uint32_t w[NT];
            if constexpr (NT == 8) {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                const uint4 b = *reinterpret_cast<const uint4 *>(src + 4);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
                w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
            } else {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
            }
            // 2-bit words hold 16 tokens: the lane's 8 are the odd or even
            // byte of each half
            const int sh = BITS == 2 ? 8 * (g & 1) : 0;
#pragma unroll
            for (int n = 0; n < NT; ++n) tv.cw[ks][n] = w[n] >> sh;
        }
        const SZT *sp = reinterpret_cast<const SZT *>(sb + kCodeBytes + sub * kSzBytes1);
        const SZT *zp = reinterpret_cast<const SZT *>(sb + kCodeBytes + kSzBytes + sub * kSzBytes1);
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            tv.s[k] = (float)sp[lane * NG + k];
            tv.z[k] = (float)zp[lane * NG + k];
        }
    }
    __device__ static void init(State &st) {
        st.bias = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kMfmaRows; ++r)
#pragma unroll
            for (int k = 0; k < NG; ++k) st.zs[r][k] = 0.f;
    }
    __device__ static void pv(Tile &tv, State &st, f32x4 (&acc)[NT], const float (&p)[kMfmaRows],
                              const float (&corr)[kMfmaRows], bool rescale, int n_in, _Float16 *pw16,
                              int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        uint16_t *pw = reinterpret_cast<uint16_t *>(pw16);
        float s[NG], z[NG];
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            s[k] = tv.s[k];
            z[k] = tv.z[k];
        }
        if (n_in < kWave) {  // tokens past the split end: p = 0, s and z possibly unwritten
            const bool ok = lane < n_in;
#pragma unroll
            for (int k = 0; k < NG; ++k) {
                s[k] = ok ? s[k] : 0.f;
                z[k] = ok ? z[k] : 0.f;
            }
        }
        if (rescale) {  // some row's running max moved
            const f32x4 cv4 = f32x4{corr[0], corr[1], corr[2], corr[3]};
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= cv4;
            // bias rows 4*(lane/16) + i belong to query row i
            st.bias *= cv4;
#pragma unroll
            for (int r = 0; r < kMfmaRows; ++r)
#pragma unroll
                for (int k = 0; k < NG; ++k) st.zs[r][k] *= corr[r];
        }
        // 2-bit codes: operand dwords 1 and 2 of a lane's 8 tokens take
        // their codes in place, at mantissa bits 2-3 and 4-5 (128 + 4c and
        // 128 + 16c, still exact); those tokens' weights carry the inverse
        // power of two, so every product is unchanged
        float sw[NG];
#pragma unroll
        for (int k = 0; k < NG; ++k) sw[k] = s[k];
        if constexpr (BITS == 2) {
            const int jt = (lane >> 1) & 3;  // dword of this token within its operand
            const float f = jt == 1 ? 0.25f : (jt == 2 ? 0.0625f : 1.f);
#pragma unroll
            for (int k = 0; k < NG; ++k) sw[k] = s[k] * f;
        }
        // w = p * s as bf16 hi + lo (both round to nearest), two rows at a time
#pragma unroll
        for (int k = 0; k < NG; ++k) {
#pragma unroll
            for (int r = 0; r < kMfmaRows; r += 2) {
                const float w0 = p[r] * sw[k], w1 = p[r + 1] * sw[k];
                const uint32_t hi = bf16x2_rn(w0, w1);
                const float l0 = w0 - __uint_as_float(hi << 16);
                const float l1 = w1 - __uint_as_float(hi & 0xffff0000u);
                const uint32_t lo = bf16x2_rn(l0, l1);
                pw[(8 * k + r) * kPStride + lane] = (uint16_t)hi;
                pw[(8 * k + r + 1) * kPStride + lane] = (uint16_t)(hi >> 16);
                pw[(8 * k + 4 + r) * kPStride + lane] = (uint16_t)lo;
                pw[(8 * k + 4 + r + 1) * kPStride + lane] = (uint16_t)(lo >> 16);
                st.zs[r][k] = fmaf(p[r], z[k], st.zs[r][k]);
                st.zs[r + 1][k] = fmaf(p[r + 1], z[k], st.zs[r + 1][k]);
            }
        }
        wave_lds_sync();
        const uint32_t cm = opaque_u32(kCodeMask), cbias = opaque_u32(kBias);
        const uint32_t cm2 = opaque_u32(kCodeMask << 2), cm4 = opaque_u32(kCodeMask << 4);
        const bf16x8 b128 = __builtin_bit_cast(bf16x8, make_uint4(cbias, cbias, cbias, cbias));
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            // A lane l: row l%16, tokens 32ks + 8(l/16) .. +7
            const bf16x8 a = *reinterpret_cast<const bf16x8 *>(pw + l16 * kPStride + 32 * ks + 8 * g);
            st.bias = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b128, st.bias, 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const uint32_t y = tv.cw[ks][n];
                uint32_t d4[4];
                if constexpr (BITS == 2) {
                    d4[0] = (y & cm) | cbias;
                    d4[1] = (y & cm2) | cbias;
                    d4[2] = (y & cm4) | cbias;
                    d4[3] = ((y >> 6) & cm) | cbias;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) d4[j] = ((y >> (BITS * j)) & cm) | cbias;
                }
                const bf16x8 bop = __builtin_bit_cast(bf16x8, make_uint4(d4[0], d4[1], d4[2], d4[3]));
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bop, acc[n], 0, 0, 0);
            }
        }
        wave_lds_sync();
    }
    // acc[n] of lane l holds rows 4(l/16) .. +3 of dim 8(l%16) + n; rows
    // 8g + 0..3 (hi) and 8g + 4..7 (lo) are group g's, so lanes 32g .. 32g+31
    // carry the dims of group g.  The hi part also carries sum p*z of its
    // (row, group).
    __device__ static void to_lds(const f32x4 (&acc)[NT], const State &st, float *wa, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        float zsum[NG][kMfmaRows];
#pragma unroll
        for (int k = 0; k < NG; ++k) {
            float zv_[kMfmaRows];
#pragma unroll
            for (int r = 0; r < kMfmaRows; ++r) zv_[r] = st.zs[r][k];
            wave_sum4_dpp(zv_, zsum[k]);
        }
        const int k = (NT * l16) / kGroup;  // the group of this lane's dims
        if ((g >> 1) == k) {
            const int hl = g & 1;
#pragma unroll
            for (int r = 0; r < kMfmaRows; ++r) {
                const float zr = hl != 0 ? 0.f : (NG == 2 && k == 1 ? zsum[NG - 1][r] : zsum[0][r]);
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    wa[(hl * kMfmaRows + r) * D + NT * l16 + n] = acc[n][r] - st.bias[r] + zr;
            }
        }
    }
};

// VGil for one decode step of a hybrid cache (float16 buffer) that also moves
// its tokens: the cache holds t_kv compressed tokens and a buffer window of
// n_flush + n_rem tokens (rows 0 .. at kbuf / vbuf, [b*buf_sb + h*buf_sh +
// row*buf_st + dim]); the step's n_new tokens arrive at knew / vnew.  The
// reference appends them to the buffer and flushes its n_flush oldest tokens
// into compressed storage (cache.py:656-710), then attends everything
// (attention.py:307-350).  Here one launch does both: the last split encodes
// the flushed keys (the step encode of VIl8Step), quantises their values with
// the grouped min/max rule and attends them in that compressed form at
// positions t_kv .., while every split attends its share of the t_buf =
// n_rem + n_new exact tokens (the buffer rows n_flush .., then the new
// tokens) after them; the last split of row group 0 of each (batch, KV head)
// stores the flushed tokens' index rows, codes, scales and zeros at
// positions t_kv .. and the new tokens at buffer rows n_flush + n_rem ..
template <int D, int BITS, int NG, class SZT>
struct VGilStep : VGil<D, BITS, NG, SZT> {
    struct Args : VGil<D, BITS, NG, SZT>::Args {
        const void *knew, *vnew;  // float16 [b*new_sb + h*new_sh + j*new_st + dim]
        int64_t new_sb, new_sh, new_st, n_rem, n_flush;
        const float *centroids;  // [n_blocks][n_centroids][8] float32
        const float *cb_norms;   // |C|^2 per prepared codebook lane (ss_codebook_f16x2)
        uint8_t *idx_out;        // the index cache the kernel reads (c.idx)
        uint32_t *codes_out;     // the code words (codes)
        SZT *scales_out, *zeros_out;
        void *kput, *vput;       // the buffer stores at the window (kbuf / vbuf)
    };
    static constexpr bool kStepShare = true;
    static constexpr bool kHybridStep = true;
    static constexpr bool kStepQuant = true;  // the flushed values are quantised
    static constexpr bool kHeavyCapable = false;
    static constexpr int kBits = BITS;
    static constexpr int kNG = NG;
    using SzT = SZT;
};

// The grouped min/max quantisation of one token's values (reference
// kernels.py:1173-1228: scale = (max - min) / (2^bits - 1), at least 1e-8;
// code = clamp(round((x - min) / scale)), the same IEEE steps as
// values.hip's quantize_grouped_kernel), the wave holding dims lane + 64k:
// codes q[k], and the scale and zero of dim lane + 64k's group.
template <int D, int BITS, int NG>
__device__ __forceinline__ void quantize_token_wave(const float (&x)[D / kWave], float (&q)[D / kWave],
                                                    float (&sc)[D / kWave], float (&mn)[D / kWave]) {
    constexpr int DL = D / kWave;
    constexpr int G = D / NG;                  // group size: 32, 64 or 128
    constexpr int SPAN = G < kWave ? G : kWave;  // lanes of one group per k
    constexpr float maxv = (float)((1 << BITS) - 1);
    float lo[DL], hi[DL];
#pragma unroll
    for (int k = 0; k < DL; ++k) lo[k] = hi[k] = x[k];
    if constexpr (G > kWave) {  // one group spans every k (G = 128 = D)
        float a = lo[0], b = hi[0];
#pragma unroll
        for (int k = 1; k < DL; ++k) {
            a = fminf(a, lo[k]);
            b = fmaxf(b, hi[k]);
        }
#pragma unroll
        for (int k = 0; k < DL; ++k) {
            lo[k] = a;
            hi[k] = b;
        }
    }
#pragma unroll
    for (int o = SPAN / 2; o > 0; o >>= 1)
#pragma unroll
        for (int k = 0; k < DL; ++k) {
            lo[k] = fminf(lo[k], __shfl_xor(lo[k], o));
            hi[k] = fmaxf(hi[k], __shfl_xor(hi[k], o));
        }
#pragma unroll
    for (int k = 0; k < DL; ++k) {
        float s = __fdiv_rn(__fsub_rn(hi[k], lo[k]), maxv);
        if (s < 1e-8f) s = 1e-8f;
        const float qf = rintf(__fdiv_rn(__fsub_rn(x[k], lo[k]), s));
        q[k] = fminf(fmaxf(qf, 0.f), maxv);
        sc[k] = s;
        mn[k] = lo[k];
    }
}

// TurboQuant 2-bit values (reference value_codecs.py:136-177) on the matrix
// cores: per token a norm and 2-bit codes of the rotated unit vector, held
// token-interleaved as VGil's words ([cap/16][D] per (b, h)); norms [cap].
// The value is norm * L(code) with the four Lloyd-Max levels L ascending.  A
// symmetric table is affine in the two code bits:
//   L(c) = L0 + (L1 - L0) c + (L2 - 2 L1 + L0) bit1(c)        (L3 = L2 + L1 - L0)
// so P.V = L0 sum w + (L1 - L0) sum w c + (L2 - 2 L1 + L0) sum w bit1 with
// w = p * norm: VGil's products (A = w as bf16 hi/lo rows, B = 128 + code)
// give sum w c, one more product per (k-step, N-tile) with B = 128 + 2 bit1
// (the bit left in place, the same per-token powers of two as the codes)
// gives sum w bit1 into rows 8-15 of the same accumulator (A rows 0-7
// repeated as rows 8-15, each half zero in the other product), and sum w
// accumulates in fp32 on the lanes.  The accumulation is in the rotated
// basis; the rotation is applied per output row after the merge
// (transformed_decode).
template <int D>
struct VTq {
    struct Args {
        const uint32_t *codes;  // token-interleaved 2-bit words
        const float *norms;     // [rows]
        float l0, l1, l2;       // levels L0, L1 - L0, L2 - 2 L1 + L0
    };
    static constexpr int NT = D / 16;
    static constexpr int BITS = 2, TPW = 16;
    static constexpr int kCodeBytes1 = kWave * D * BITS / 8;  // 2 KB at D = 128
    static constexpr int kSzBytes1 = kWave * 4;               // the 64 norms
    static constexpr bool kPrivateRing = true;
    static constexpr int kSub = 1;
    static constexpr int kCodeBytes = kCodeBytes1;
    static constexpr int kSzBytes = kSzBytes1;
    static constexpr bool kHybridBuffer = false;  // the buffer joins as its own rotated partial
    static constexpr bool kHeavyCapable = true;
    static constexpr int kTileV = kCodeBytes + 1024;
    static constexpr int kLoadsV = kCodeBytes / 1024 + 1;
    static constexpr int kPRows = 16;
    static constexpr int kMaxSlots = 16;
    static constexpr int kComputeWaves = 8;
    static constexpr uint32_t kCodeMask = 0x00030003u;
    static constexpr uint32_t kBit1Mask = 0x00020002u;
    static constexpr uint32_t kBias = 0x43004300u;  // two bf16 128.0
    static_assert(NT == 8 || NT == 4, "n-tiles");
    struct Tile {
        uint32_t cw[2][NT];  // as VGil: the lane's 8 tokens of dims 8*(lane%16) + n
        float n;             // norm of token `lane`
    };
    static constexpr bool kRegUnits = true;
    static constexpr float kMaxLag = 8.f;  // bf16 hi/lo probabilities
    struct Raw {
        uint32_t cw[2][NT];
        float n;
    };
    __device__ static void load(Raw &u, const Args &a, int64_t bh, int64_t cap, int64_t t0, int64_t t_last,
                                int lane) {
        load_code_words<D, NT, TPW>(u.cw, a.codes, bh, cap, t0, t_last, lane);
        u.n = a.norms[bh * cap + min(t0 + lane, t_last)];
    }
    __device__ static void from_raw(Tile &tv, const Raw &u, int lane) {
        const int sh = 8 * ((lane >> 4) & 1);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
            for (int n = 0; n < NT; ++n) tv.cw[ks][n] = u.cw[ks][n] >> sh;
        tv.n = u.n;
    }
    struct State {
        f32x4 bias;          // 128 * sum of the staged A rows, laid out as acc
        float ws[kMfmaRows]; // sum of p * norm of this lane's tokens
    };
    __device__ static void issue(const Args &a, int64_t bh, int64_t cap, int64_t t0, int64_t t_last,
                                 uint32_t sb, int lane) {
        const char *chead = reinterpret_cast<const char *>(a.codes + bh * (cap / TPW) * D);
        const char *np = reinterpret_cast<const char *>(a.norms + bh * cap + t0);
        const int64_t wb0 = t0 / TPW;
        if (t0 + kWave - 1 <= t_last) {
            const char *cb = chead + wb0 * D * 4;
#pragma unroll
            for (int i = 0; i < kCodeBytes / 1024; ++i)
                __builtin_amdgcn_global_load_lds(cb + (uint32_t)(i * 1024 + lane * 16),
                                                 reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                                 kCpolNt);
            if (lane < kSzBytes / 16)
                __builtin_amdgcn_global_load_lds(np + lane * 16,
                                                 reinterpret_cast<lds_t<void> *>(sb + kCodeBytes), 16, 0,
                                                 kCpolNt);
            return;
        }
        // past the split's last token: code chunks clamp to its block, norm
        // chunks to the one holding it
        const int64_t blk_last = t_last / TPW;
#pragma unroll
        for (int i = 0; i < kCodeBytes / 1024; ++i) {
            const int w = (i * kWave + lane) * 4;
            const int64_t blk = min(wb0 + w / D, blk_last);
            __builtin_amdgcn_global_load_lds(chead + (blk * D + w % D) * 4,
                                             reinterpret_cast<lds_t<void> *>(sb + i * 1024), 16, 0,
                                             kCpolNt);
        }
        const int64_t ch_last = (t_last - t0) / 4;
        if (lane < kSzBytes / 16)
            __builtin_amdgcn_global_load_lds(np + min((int64_t)lane, ch_last) * 16,
                                             reinterpret_cast<lds_t<void> *>(sb + kCodeBytes), 16, 0,
                                             kCpolNt);
    }
    __device__ static void copy(Tile &tv, const char *sb, int sub, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int tk = 32 * ks + 8 * g;
            const uint32_t *src = reinterpret_cast<const uint32_t *>(sb) + (tk / TPW) * D + (NT * l16) % D;
            uint32_t w[NT];
            if constexpr (NT == 8) {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                const uint4 b = *reinterpret_cast<const uint4 *>(src + 4);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
                w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
            } else {
                const uint4 a = *reinterpret_cast<const uint4 *>(src);
                w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
            }
            const int sh = 8 * (g & 1);  // the lane's 8 tokens: odd or even byte of each half
#pragma unroll
            for (int n = 0; n < NT; ++n) tv.cw[ks][n] = w[n] >> sh;
        }
        tv.n = reinterpret_cast<const float *>(sb + kCodeBytes)[lane];
        (void)sub;
    }
    __device__ static void init(State &st) {
        st.bias = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int r = 0; r < kMfmaRows; ++r) st.ws[r] = 0.f;
    }
    __device__ static void pv(Tile &tv, State &st, f32x4 (&acc)[NT], const float (&p)[kMfmaRows],
                              const float (&corr)[kMfmaRows], bool rescale, int n_in, _Float16 *pw16,
                              int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        uint16_t *pw = reinterpret_cast<uint16_t *>(pw16);
        float s = tv.n;
        if (n_in < kWave) s = lane < n_in ? s : 0.f;  // past the split end: p = 0, norm unwritten
        if (rescale) {
            const f32x4 cv4 = f32x4{corr[0], corr[1], corr[2], corr[3]};
#pragma unroll
            for (int n = 0; n < NT; ++n) acc[n] *= cv4;
            st.bias *= cv4;
#pragma unroll
            for (int r = 0; r < kMfmaRows; ++r) st.ws[r] *= corr[r];
        }
#pragma unroll
        for (int r = 0; r < kMfmaRows; ++r) st.ws[r] = fmaf(p[r], s, st.ws[r]);
        // the codes of dwords 1 and 2 of a lane's 8 tokens stay in place
        // (x4, x16): those tokens' weights carry 1/4 and 1/16 (as VGil)
        const int jt = (lane >> 1) & 3;
        const float sw = s * (jt == 1 ? 0.25f : (jt == 2 ? 0.0625f : 1.f));
#pragma unroll
        for (int r = 0; r < kMfmaRows; r += 2) {
            const float w0 = p[r] * sw, w1 = p[r + 1] * sw;
            const uint32_t hi = bf16x2_rn(w0, w1);
            const float l0 = w0 - __uint_as_float(hi << 16);
            const float l1 = w1 - __uint_as_float(hi & 0xffff0000u);
            const uint32_t lo = bf16x2_rn(l0, l1);
            pw[r * kPStride + lane] = (uint16_t)hi;
            pw[(r + 1) * kPStride + lane] = (uint16_t)(hi >> 16);
            pw[(4 + r) * kPStride + lane] = (uint16_t)lo;
            pw[(4 + r + 1) * kPStride + lane] = (uint16_t)(lo >> 16);
        }
        wave_lds_sync();
        const uint32_t cm = opaque_u32(kCodeMask), cbias = opaque_u32(kBias);
        const uint32_t cm2 = opaque_u32(kCodeMask << 2), cm4 = opaque_u32(kCodeMask << 4);
        const uint32_t bm = opaque_u32(kBit1Mask), bm2 = opaque_u32(kBit1Mask << 2),
                       bm4 = opaque_u32(kBit1Mask << 4);
        const bf16x8 b128 = __builtin_bit_cast(bf16x8, make_uint4(cbias, cbias, cbias, cbias));
        // A rows 0-7 (hi, lo of the four query rows) multiply the codes, the
        // same rows repeated as A rows 8-15 multiply the high code bits: one
        // accumulator holds both sums (rows 8-15 of acc are the bit-1 sums)
        const bool top = l16 < 8;
        const uint4 zero4 = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const uint4 av = *reinterpret_cast<const uint4 *>(pw + (l16 & 7) * kPStride + 32 * ks + 8 * g);
            const bf16x8 a = __builtin_bit_cast(bf16x8, av);
            const bf16x8 a_c = __builtin_bit_cast(bf16x8, top ? av : zero4);
            const bf16x8 a_b = __builtin_bit_cast(bf16x8, top ? zero4 : av);
            st.bias = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b128, st.bias, 0, 0, 0);
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const uint32_t y = tv.cw[ks][n];
                const uint32_t y6 = y >> 6;
                const bf16x8 bc = __builtin_bit_cast(
                    bf16x8, make_uint4((y & cm) | cbias, (y & cm2) | cbias, (y & cm4) | cbias, (y6 & cm) | cbias));
                const bf16x8 bb = __builtin_bit_cast(
                    bf16x8, make_uint4((y & bm) | cbias, (y & bm2) | cbias, (y & bm4) | cbias, (y6 & bm) | cbias));
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_c, bc, acc[n], 0, 0, 0);
                acc[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_b, bb, acc[n], 0, 0, 0);
            }
        }
        wave_lds_sync();
    }
    // acc rows 0-3 (lanes 0-15) hold the hi parts, rows 4-7 (lanes 16-31)
    // the lo parts of the four query rows: acc - bias = sum w c; rows 8-15
    // (lanes 32-63) the same parts of sum w (2 bit1) + bias (the A rows carry
    // w times the in-place powers of two, the bias the same).  Each lane
    // scales its part by L1 - L0 or (L2 - 2 L1 + L0) / 2 and lanes 0-31 add
    // the bit-1 part of lane + 32.  The L0 sum w term, from the lanes' fp32
    // sums of p * norm, goes with the hi part.
    __device__ static void to_lds_args(const f32x4 (&acc)[NT], const State &st, const Args &a, float *wa,
                                       int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        float wsum[kMfmaRows];
        wave_sum4_dpp(st.ws, wsum);
        const float f = g < 2 ? a.l1 : a.l2 * 0.5f;
#pragma unroll
        for (int r = 0; r < kMfmaRows; ++r) {
            const float bz = st.bias[r];
            const float c0 = g == 0 ? a.l0 * wsum[r] : 0.f;
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                const float v = f * (acc[n][r] - bz);
                const float vb = __shfl_xor(v, 32);
                if (g < 2) wa[(g * kMfmaRows + r) * D + NT * l16 + n] = c0 + v + vb;
            }
        }
    }
};

template <int D, int NC, class VF>
__global__ void __launch_bounds__((VF::kPrivateRing ? NC : NC + 1) * kWave)
    decode_attn_mfma_kernel(DecodeCommon c, typename VF::Args va) {
    using K = WsCfg<D, NC, VF>;
    constexpr int R = kMfmaRows;
    constexpr int NB = K::kNB;
    constexpr int NT = D / 16;  // MFMA N-tiles (16 dims each)
    constexpr int THREADS = K::kWaves * kWave;
    constexpr int LPT = K::kLoadsPerTile;

    extern __shared__ __align__(16) float4 smem4[];
    char *smem = reinterpret_cast<char *>(smem4);
    float4 *lut4 = smem4;                                              // [NB][256]
    _Float16 *pst = reinterpret_cast<_Float16 *>(smem + K::kLut);     // [NC][kPRows][kPStride]
    volatile lds_t<int> *ready = to_lds<int>(smem + K::kLut + K::kPst);
    volatile lds_t<int> *done = ready + K::kFlagWords;               // [slot][sub]
    volatile lds_t<int> *cbar = done + K::kFlagWords * K::kSub;  // compute-wave barrier counter
    char *ring = smem + K::kRing;
    // buffer partial: m [R], l [R], acc [R][D] (acc holds the query copy
    // until the share is done)
    float *bpart = reinterpret_cast<float *>(smem + K::kLut + K::kPst + K::kFlags);
    // a fused step's new tokens' index rows [kMaxStepTokens][NB] (the step
    // share scores them from the LUT)
    uint8_t *step_idx = reinterpret_cast<uint8_t *>(smem + K::kLut + K::kPst + K::kFlags + K::kBufPart);
    // and the encode's per-wave candidates [NC][4 blocks][4 tokens]
    f32x4 *step_part = reinterpret_cast<f32x4 *>(step_idx + 64);
    // 16-byte LUT reads through the LDS object itself (an address-space
    // cast the compiler folds to the constant LDS address)
    const lds_t<f32x4> *lut_l = (const lds_t<f32x4> *)smem4;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    // wave-uniform (scalar) wave index: all tile control flow stays scalar
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool loader = !K::kPriv && wv == NC;
    const int col = blockIdx.y;
    const int split = blockIdx.x;
    const int rg = col % c.n_rg;
    const int kvh = (col / c.n_rg) % c.n_kv_heads;
    const int64_t bb = col / (c.n_rg * c.n_kv_heads);
    const int64_t bh = bb * c.n_kv_heads + kvh;
    auto row_off = [&](int r) -> int64_t {
        const int64_t g = (int64_t)rg * R + r;
        const int64_t rr = g / c.t_q, tq = g - rr * c.t_q;
        return ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
    };
    auto row_ok = [&](int r) -> bool { return (int64_t)rg * R + r < c.rows_total; };

    const int64_t span = (int64_t)c.tiles_per_split * kWave + c.split_pad;
    const int64_t t_beg = (int64_t)split * span;
    const int64_t t_end = min(c.t_kv, t_beg + span);
    // 64-token units (one per compute step) and ring tiles of kSub units
    const int n_units = t_end > t_beg ? (int)((t_end - t_beg + kWave - 1) / kWave) : 0;
    const int n_tiles = (n_units + K::kSub - 1) / K::kSub;
    const uint8_t *idx_head = c.idx + bh * c.cap * NB;
    const int64_t t_last = max(t_end - 1, (int64_t)0);
    const int g = lane >> 4, l16 = lane & 15;
    // this split's share of the token buffer (wave-uniform)
    int64_t t_buf = 0;
    if constexpr (VF::kHybridBuffer) t_buf = va.t_buf;
    constexpr bool kStep = StepShareOf<VF>::value;     // a fused step encodes tokens
    constexpr bool kHStep = HybridStepOf<VF>::value;   // ... beside a share of exact tokens
    constexpr bool kStepOnly = kStep && !kHStep;       // ... that are its whole share
    // (a fused step's new tokens all go to the last split; a hybrid step's
    // exact tokens are shared out as a hybrid cache's buffer)
    const int64_t bshare = kStepOnly ? t_buf : (t_buf + c.n_splits - 1) / c.n_splits;
    const int64_t bj0 = kStepOnly ? 0 : min((int64_t)split * bshare, t_buf);
    const int64_t bj1 = kStepOnly ? (split == c.n_splits - 1 ? t_buf : 0) : min(bj0 + bshare, t_buf);
    // tokens the split encodes (and scores from the LUT): a step's new
    // tokens, or a hybrid step's flushed ones, all in the last split
    int n_step = 0;
    if constexpr (kStepOnly) n_step = (int)bj1;
    if constexpr (kHStep) n_step = split == c.n_splits - 1 ? (int)va.n_flush : 0;
    // the split's share of exact (buffered or new) tokens
    const bool has_ex = VF::kHybridBuffer && !kStepOnly && bj1 > bj0;
    const bool has_buf = VF::kHybridBuffer && (bj1 > bj0 || n_step > 0);

    // Barrier that orders LDS only: a wave's outstanding global loads (the
    // loader's tile copies) do not have to land first, which __syncthreads'
    // workgroup release fence would require.
    auto lds_barrier = [] {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };
    // A bounded wait gave up: record which kind in the sticky word (one
    // vector atomic per wave; the host reads and clears it).
    auto wait_gave_up = [&](unsigned kind) {
        if (lane == 0) {
            __hip_atomic_fetch_or(c.wait_fail, kind, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(c.wait_host, kind, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    };
    // Barrier among the NC compute waves only (the loader never joins it):
    // each wave adds 1 to an LDS counter once its LDS writes are done and
    // waits until all NC waves have arrived for this phase (bounded wait).
    auto compute_barrier = [&](int phase) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if (lane == 0) __hip_atomic_fetch_add(const_cast<lds_t<int> *>(cbar), 1, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_WORKGROUP);
        int spins = 0;
        while (*cbar < phase * NC) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > c.spin_limit) {
                wait_gave_up(kWaitBarrier);
                break;
            }
        }
        asm volatile("" ::: "memory");
    };

    // Loader: ring tile j (tokens t_beg + 64*kSub*j ..) into slot j % kSlots:
    // the value format's copies, then the index rows (contiguous, chunks past
    // the one holding the split's last token clamp to it), so every load
    // stays in bounds.  The LDS destination of lane l is M0 + 16*l.
    auto issue_at = [&](int j, uint32_t sb) {
        const int64_t t0 = t_beg + (int64_t)j * K::kSub * kWave;
        VF::issue(va, bh, c.cap, t0, t_last, sb, lane);
        const uint8_t *ip = idx_head + t0 * NB;
        const bool full = t0 + K::kSub * kWave - 1 <= t_last;
        const int64_t ch_last = ((t_last - t0) * NB) / 16;
#pragma unroll
        for (int i = 0; i < K::kLoadsI; ++i) {
            const int ch = i * kWave + lane;
            if (K::kTileI % 1024 == 0 || ch * 16 < K::kTileI) {
                const uint8_t *src = full ? ip + (uint32_t)(ch * 16) : ip + min((int64_t)ch, ch_last) * 16;
                __builtin_amdgcn_global_load_lds(
                    src, reinterpret_cast<lds_t<void> *>(sb + K::kTileV + i * 1024), 16, 0, kCpolNt);
            }
        }
    };
    const uint32_t ring_l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(ring));
    auto issue = [&](int j) { issue_at(j, ring_l + (uint32_t)((j % K::kSlots) * K::kSlot)); };
    // private rings: slot s of this wave
    auto priv_slot = [&](int s) { return (uint32_t)((wv * K::kPrivSlots + s) * K::kSlot); };
    int nq = 0;  // private rings: units this wave has issued
    int issued = 0, landed = 0;
    // register units: a wave's unit u (index row, value data, heavy key
    // dims of token `lane`) loaded into one of two register sets, the next
    // unit's loads issued before the current one is computed
    constexpr bool kRegs = VfRegUnits<VF>::value;
    constexpr float kLag = VfMaxLag<VF>::value;
    constexpr bool HV = VfHeavyMfma<VF>::value;
    constexpr int HVN = HV ? kMaxHeavyMfma / 8 : 1;
    struct RegUnit {
        IdxRow<NB> ir;
        typename RawUnitOf<VF, kRegs>::type raw;
        uint4 khv[HVN];
    };
    auto load_ru = [&](RegUnit &x, int u) {
        if constexpr (kRegs) {
            const int64_t t0 = t_beg + (int64_t)u * kWave;
            const int64_t tk = min(t0 + lane, t_last);
            x.ir.load(c.idx + (bh * c.cap + tk) * NB, true);
            VF::load(x.raw, va, bh, c.cap, t0, t_last, lane);
            if constexpr (HV) {
                if (c.nhd > 0) {
                    const uint4 *hp = reinterpret_cast<const uint4 *>(c.kheavy + (bh * c.cap + tk) * c.nhd);
#pragma unroll
                    for (int j8 = 0; j8 < HVN; ++j8)
                        if (8 * j8 < c.nhd) x.khv[j8] = hp[j8];
                }
            }
        }
    };
    RegUnit ua, ub;
    // Wave w takes units w, w + NC, ... of the split.  Where wave 0 first
    // attends the split's share of buffered tokens (and, in a hybrid step,
    // scores the flushed tokens), it skips its first share_skip units, which
    // waves 1, 2, ... take after their own: a fixed schedule (the sums, and so
    // the results, never depend on timing) that evens out the waves' ends.
    int share_skip = 0;
    if constexpr (kRegs && VF::kHybridBuffer) {
        if (has_ex) share_skip += kShareSkipRounds;
        if (n_step > 0) share_skip += kStepSkipRounds;
    }
    const int n_own = wv < n_units ? (n_units - wv + NC - 1) / NC : 0;
    auto unit_of = [&](int i) -> int {  // this wave's i-th unit (n_units: none)
        if (wv == 0) {
            const int u = (i + share_skip) * NC;
            return u < n_units ? u : n_units;
        }
        if (i < n_own) return wv + i * NC;
        const int j = (wv - 1) + (i - n_own) * (NC - 1);  // wave 0's skipped unit j * NC
        return (j < share_skip && j * NC < n_units) ? j * NC : n_units;
    };

    // Prologue.  The compute waves' small loads (query element, permutation
    // entry, codebook entries) are issued before the loader's first tiles, so
    // they sit ahead of the tiles in the compute unit's memory queue; the
    // LUT is built while the first tiles are in flight.
    constexpr int LT = K::kLutTiles;  // LUT tiles (4 blocks x 16 centroids) per compute wave
    float *qraw = reinterpret_cast<float *>(pst);  // [R][D] (P staging is free here)
    float *qp = qraw + R * D;                      // [R][D]
    constexpr int CT = NC * kWave;             // compute threads
    constexpr int QE = (R * D + CT - 1) / CT;  // query elements per compute thread
    if (tid < K::kFlagWords * (1 + K::kSub)) ready[tid] = -1;  // ready[] and done[][]
    if (tid == 0) {
        cbar[0] = 0;
        cbar[2] = 0;   // hybrid step: block groups whose flushed tokens' indices are decided
    }
    int64_t lim[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t gr = (int64_t)rg * R + r;
        lim[r] = !row_ok(r) ? -1 : (c.causal ? c.q_offset + (gr % c.t_q) : INT64_MAX);
    }
    // last token every live row sees
    int64_t lim_min = INT64_MAX;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (row_ok(r)) lim_min = min(lim_min, lim[r]);
    f32x4 acc[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    typename VF::State vst;
    VF::init(vst);
    // running maxima; a row past the last query row gets a maximum no score
    // reaches, so its probabilities are 0 and it never forces a reduction
    float m[R], lsum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = row_ok(r) ? -1e30f : 3e38f;
        lsum[r] = 0.f;
    }

    // The two roles run in separate branches up to the end of the tile loop
    // (one shared LDS-only barrier, then compute-only barriers), so no code
    // after a join inherits the loader's outstanding tile copies as pending
    // loads, and the loader streams from the start without waiting for the
    // LUT.
    // Hybrid caches: compute wave 0 attends this split's share of the token
    // buffer (positions t_kv + bj0 ..) with fp32 dot products against the
    // unpermuted scaled query, before its tiles; the share's (m, l, acc)
    // join the workgroup combine as one more wave.  Keys in log2 units, as
    // the LUT.
    // a fused step's new tokens (the last split): key and value dims
    // lane + 64k of each, loaded in the prologue
    constexpr int DLs = kStep ? D / kWave : 1;
    constexpr int NS = kStep ? kMaxStepTokens : 1;
    float kpre[NS][DLs], vpre[NS][DLs];
    // A hybrid cache's share of at most kShareRegs 16-bit buffered tokens
    // (wave 0): their key and value dims lane + 64k, loaded in the prologue
    // too (the heavy-dim kernels have no registers to spare)
    constexpr bool kShPre = VF::kHybridBuffer && !kStepOnly && !HV;
    constexpr int kShareRegs = 8;
    constexpr int NSH = kShPre ? kShareRegs : 1;
    constexpr int DLh = kShPre ? D / kWave : 1;
    unsigned short hk_raw[NSH][DLh], hv_raw[NSH][DLh];
    const int n_sh = (int)(bj1 - bj0);
    bool sh_pre = false, sh_lds = false;
    if constexpr (kShPre) {
        const bool b16 = va.buf_dtype == SS_F16 || va.buf_dtype == SS_BF16;
        sh_pre = has_ex && wv == 0 && n_sh <= kShareRegs && b16;
        sh_lds = has_ex && n_sh > kShareRegs && n_sh <= K::kShareLdsTok && b16;
    }
    // Exact token j of the share (its key or value row): buffer row j; in a
    // hybrid step buffer row n_flush + j for the n_rem buffered tokens that
    // stay, then the step's new tokens (float16, checked on the host).  Its
    // position is ex_pos0 + j.
    auto ex_row = [&](const auto &bv, bool is_v, int64_t j) -> const char * {
        if constexpr (kHStep) {
            if (j >= bv.n_rem)
                return static_cast<const char *>(is_v ? bv.vnew : bv.knew) +
                       (bb * bv.new_sb + kvh * bv.new_sh + (j - bv.n_rem) * bv.new_st) * 2;
            j += bv.n_flush;
        }
        const int64_t es = bv.buf_dtype == SS_F32 ? 4 : 2;
        return static_cast<const char *>(is_v ? bv.vbuf : bv.kbuf) +
               (bb * bv.buf_sb + kvh * bv.buf_sh + j * bv.buf_st) * es;
    };
    int64_t ex_pos0 = c.t_kv;
    if constexpr (kHStep) ex_pos0 += va.n_flush;
    // the LDS copy of the share: keys [kShareLdsTok][D], then values
    const unsigned short *sh_k = reinterpret_cast<const unsigned short *>(
        smem + K::kLut + K::kPst + K::kFlags + K::kBufPart + K::kStepLds);
    const unsigned short *sh_v = sh_k + K::kShareLdsTok * D;
    auto buffer_share = [&](const auto &bv) {
        constexpr int DL = D / kWave;  // value dims per lane
        float bm[R], bl[R], ba[R][DL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            bm[r] = -1e30f;
            bl[r] = 0.f;
#pragma unroll
            for (int k = 0; k < DL; ++k) ba[r][k] = 0.f;
        }
        const float *bq = bpart + 2 * R;  // [R][D] query copy
        f32x4 *pb = reinterpret_cast<f32x4 *>(pst);  // wave 0's P staging: p of 64 tokens
        const int64_t head = bb * bv.buf_sb + kvh * bv.buf_sh;
        // key / value row of exact-share token j (the buffer's own rows,
        // indexed directly, outside a hybrid step)
        auto krow_of = [&](int64_t j) -> const char * {
            if constexpr (kHStep) return ex_row(bv, false, j);
            return static_cast<const char *>(bv.kbuf) +
                   (head + j * bv.buf_st) * (bv.buf_dtype == SS_F32 ? 4 : 2);
        };
        if constexpr (kShPre) {
            if (sh_pre || sh_lds) {
                // the prefetched share (registers, or the LDS copy), eight
                // tokens at a time: each token's four scores as wave sums of
                // the lanes' partial dot products (lane: dims lane + 64k),
                // online softmax over the chunks, P.V on the lanes' dims
                if (sh_lds) wait_vmcnt<0>();  // wave 0's copies have landed
                const bool bf = bv.buf_dtype == SS_BF16;
                auto f32 = [&](unsigned short h) {
                    return bf ? __uint_as_float((uint32_t)h << 16) : __half2float(__ushort_as_half(h));
                };
                float qv[R][DLh];
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int k = 0; k < DLh; ++k) qv[r][k] = bq[r * D + lane + kWave * k];
                for (int c0 = 0; c0 < n_sh; c0 += NSH) {
                    unsigned short kc[NSH][DLh], vc[NSH][DLh];
#pragma unroll
                    for (int j = 0; j < NSH; ++j)
#pragma unroll
                        for (int k = 0; k < DLh; ++k) {
                            if (sh_lds) {
                                const int row = min(c0 + j, n_sh - 1);
                                kc[j][k] = sh_k[row * D + lane + kWave * k];
                                vc[j][k] = sh_v[row * D + lane + kWave * k];
                            } else {
                                kc[j][k] = hk_raw[j][k];
                                vc[j][k] = hv_raw[j][k];
                            }
                        }
                    float sc[NSH][R];
#pragma unroll
                    for (int j = 0; j < NSH; ++j) {
                        float part[R];
#pragma unroll
                        for (int r = 0; r < R; ++r) {
                            part[r] = 0.f;
#pragma unroll
                            for (int k = 0; k < DLh; ++k) part[r] = fmaf(qv[r][k], f32(kc[j][k]), part[r]);
                        }
                        wave_sum4_dpp(part, sc[j]);
                        const int64_t pos = ex_pos0 + bj0 + c0 + j;
#pragma unroll
                        for (int r = 0; r < R; ++r)
                            sc[j][r] = (c0 + j < n_sh && pos <= lim[r]) ? sc[j][r] * kLog2e : -INFINITY;
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        float mx = sc[0][r];
#pragma unroll
                        for (int j = 1; j < NSH; ++j) mx = fmaxf(mx, sc[j][r]);
                        if (mx == -INFINITY) continue;  // nothing visible in this chunk
                        const float mn = fmaxf(bm[r], mx);
                        const float corr = fast_exp2(bm[r] - mn);
                        bm[r] = mn;
                        bl[r] *= corr;
#pragma unroll
                        for (int k = 0; k < DLh; ++k) ba[r][k] *= corr;
#pragma unroll
                        for (int j = 0; j < NSH; ++j) {
                            const float pj = fast_exp2(sc[j][r] - mn);
                            bl[r] += pj;
#pragma unroll
                            for (int k = 0; k < DLh; ++k) ba[r][k] = fmaf(pj, f32(vc[j][k]), ba[r][k]);
                        }
                    }
                }
            }
        }
        for (int64_t j0 = (sh_pre || sh_lds) ? bj1 : bj0; j0 < bj1; j0 += kWave) {
            const int64_t j = j0 + lane;
            const bool ok = j < bj1;
            float sc[R] = {};
            if constexpr (kStepOnly) {
                // a new token: its encoded index row (LDS) scored from the
                // LUT, already in log2 units
                const lds_t<uint8_t> *row = to_lds<uint8_t>(step_idx) + (ok ? j : j0) * NB;
                f32x4 e = lut_l[row[0]];
#pragma unroll
                for (int b = 1; b < NB; ++b) e += lut_l[b * kLutStride + row[b]];
#pragma unroll
                for (int r = 0; r < R; ++r) sc[r] = e[r];
            } else {
                const char *krow = krow_of(ok ? j : j0);
                for (int d0 = 0; d0 < D; d0 += 8) {
                    float kx[8];
                    if (bv.buf_dtype == SS_F16) {
                        unpack16<__half>(*reinterpret_cast<const uint4 *>(
                                             reinterpret_cast<const __half *>(krow) + d0),
                                         kx);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) kx[i] = load_as_f32(krow, bv.buf_dtype, d0 + i);
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int i = 0; i < 8; ++i) sc[r] = fmaf(bq[r * D + d0 + i], kx[i], sc[r]);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) sc[r] *= kLog2e;
            }
            const int64_t pos = (kStepOnly ? c.t_kv : ex_pos0) + j;
#pragma unroll
            for (int r = 0; r < R; ++r) sc[r] = (ok && pos <= lim[r]) ? sc[r] : -INFINITY;
            float tmax[R], p[R], corr[R];
            wave_max4_dpp(sc, tmax);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float mn = fmaxf(bm[r], tmax[r]);
                corr[r] = fast_exp2(bm[r] - mn);
                p[r] = fast_exp2(sc[r] - mn);
                bm[r] = mn;
            }
            float ps[R];
            wave_sum4_dpp(p, ps);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                bl[r] = fmaf(bl[r], corr[r], ps[r]);
#pragma unroll
                for (int k = 0; k < DL; ++k) ba[r][k] *= corr[r];
            }
            pb[lane] = f32x4{p[0], p[1], p[2], p[3]};
            wave_lds_sync();
            const int nj = (int)min(bj1 - j0, (int64_t)kWave);
            // P.V over the chunk's tokens, eight at a time: their values'
            // loads (lane-contiguous dims) are all issued before the FMAs, so
            // the chunk waits on memory once per eight tokens, not per token
            auto pv = [&](auto tag) {
                using T = decltype(tag);
                const T *vb = static_cast<const T *>(bv.vbuf);
                for (int jb = 0; jb < nj; jb += 8) {
                    float vv[8][DL];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int64_t jt = j0 + min(jb + u, nj - 1);
                        const T *vr = vb + head + jt * bv.buf_st;
                        if constexpr (kHStep) vr = reinterpret_cast<const T *>(ex_row(bv, true, jt));
#pragma unroll
                        for (int k = 0; k < DL; ++k) vv[u][k] = to_f32(vr[lane + k * kWave]);
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        if (jb + u < nj) {
                            const f32x4 pj = pb[jb + u];
#pragma unroll
                            for (int k = 0; k < DL; ++k)
#pragma unroll
                                for (int r = 0; r < R; ++r) ba[r][k] = fmaf(pj[r], vv[u][k], ba[r][k]);
                        }
                    }
                }
            };
            if constexpr (kStepOnly) {
                // a fused step's values, prefetched into registers
#pragma unroll
                for (int u = 0; u < kMaxStepTokens; ++u) {
                    if (u < nj) {
                        const f32x4 pj = pb[u];
#pragma unroll
                        for (int k = 0; k < DL; ++k)
#pragma unroll
                            for (int r = 0; r < R; ++r) ba[r][k] = fmaf(pj[r], vpre[u][k], ba[r][k]);
                    }
                }
            } else if (bv.buf_dtype == SS_F16)
                pv(__half{});
            else if (bv.buf_dtype == SS_BF16)
                pv(__hip_bfloat16{});
            else
                pv(float{});
            wave_lds_sync();
        }
        if constexpr (kHStep) {
            if (n_step > 0) {
                // a hybrid step's flushed tokens in their compressed form, at
                // positions t_kv ..: scores from the LUT by their new index
                // rows (log2 units), values code * scale + zero with the
                // scale and zero rounded to their stored type.  Their index
                // rows are complete once every block group's leader has
                // signalled (bounded wait).
                int spins = 0;
                while (cbar[2] < NB / 4) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > c.spin_limit) {
                        wait_gave_up(kWaitBarrier);
                        break;
                    }
                }
                asm volatile("" ::: "memory");
                float sc[NS][R], vh[NS][DL];
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    const lds_t<uint8_t> *row = to_lds<uint8_t>(step_idx) + min(j, n_step - 1) * NB;
                    f32x4 e = lut_l[row[0]];
#pragma unroll
                    for (int b = 1; b < NB; ++b) e += lut_l[b * kLutStride + row[b]];
                    const int64_t pos = c.t_kv + j;
#pragma unroll
                    for (int r = 0; r < R; ++r) sc[j][r] = (j < n_step && pos <= lim[r]) ? e[r] : -INFINITY;
                    if constexpr (VF::kStepQuant) {
                        using SZT = typename VF::SzT;
                        float qc[DL], qs[DL], qz[DL];
                        quantize_token_wave<D, VF::kBits, VF::kNG>(vpre[j], qc, qs, qz);
#pragma unroll
                        for (int k = 0; k < DL; ++k)
                            vh[j][k] = fmaf(qc[k], (float)(SZT)qs[k], (float)(SZT)qz[k]);
                    } else {
#pragma unroll
                        for (int k = 0; k < DL; ++k) vh[j][k] = vpre[j][k];  // fp16 values as they are
                    }
                }
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    float mx = sc[0][r];
#pragma unroll
                    for (int j = 1; j < NS; ++j) mx = fmaxf(mx, sc[j][r]);
                    if (mx == -INFINITY) continue;  // none visible to this row
                    const float mn = fmaxf(bm[r], mx);
                    const float corr = fast_exp2(bm[r] - mn);
                    bm[r] = mn;
                    bl[r] *= corr;
#pragma unroll
                    for (int k = 0; k < DL; ++k) ba[r][k] *= corr;
#pragma unroll
                    for (int j = 0; j < NS; ++j) {
                        const float pj = fast_exp2(sc[j][r] - mn);
                        bl[r] += pj;
#pragma unroll
                        for (int k = 0; k < DL; ++k) ba[r][k] = fmaf(pj, vh[j][k], ba[r][k]);
                    }
                }
            }
        }
        // the query copy is no longer read: the partial takes its place
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                bpart[r] = bm[r];
                bpart[R + r] = bl[r];
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int k = 0; k < DL; ++k) bpart[2 * R + r * D + k * kWave + lane] = ba[r][k];
    };

    // the slot of ring tile j has been copied out of by all consumers of
    // tile j - kSlots
    auto slot_free = [&](int j) {
        const int s0 = (j % K::kSlots) * K::kSub;
        bool ok = true;
#pragma unroll
        for (int u = 0; u < K::kSub; ++u) ok = ok && done[s0 + u] == j - K::kSlots;
        return ok;
    };
    if (loader) {
        // the compute waves' small loads are issued (so they are ahead of
        // the tiles in the memory queue) and the flags are initialised
        lds_barrier();
        // keep kDepth tiles in flight; publish each tile once it has landed
        int spins = 0;
        while (landed < n_tiles) {
            if (issued < n_tiles && issued - landed < K::kDepth &&
                (issued < K::kSlots || slot_free(issued))) {
                asm volatile("" ::: "memory");
                issue(issued++);
                continue;
            }
            if (issued > landed) {
                wait_oldest_tile<LPT, K::kDepth>(issued - landed);
                asm volatile("" ::: "memory");
                if (lane == 0) ready[landed % K::kSlots] = landed;
                ++landed;
                continue;
            }
            __builtin_amdgcn_s_sleep(1);  // slot still held by its consumer
            if (++spins > c.spin_limit) {
                wait_gave_up(kWaitSlot);
                break;
            }
        }
    } else {
        uint4 cb_hi[LT], cb_lo[LT];
        const float cb_mul = *c.codebook_mul;
        uint32_t q_word[QE];
        int perm_v[QE];
        int64_t q_byte[QE];
        {
            // query elements e = tid + u*CT (row e / D, dim e % D: the aligned
            // dword holding each) with their permutation entries, and the
            // codebook entries of this thread's LUT slice; loads are
            // unconditional (dummy addresses when unused)
            const int q_es = c.q_dtype == SS_F32 ? 4 : 2;
#pragma unroll
            for (int u = 0; u < QE; ++u) {
                const int e = tid + u * CT, er = e / D, ej = e - (e / D) * D;
                const bool live = e < R * D && row_ok(er);
                q_byte[u] = live ? (row_off(er) + ej) * q_es : 0;
                q_word[u] = *reinterpret_cast<const uint32_t *>(static_cast<const char *>(c.q) +
                                                                (q_byte[u] & ~int64_t(3)));
                const int *pp = c.perm ? c.perm + (e < R * D ? ej : 0)
                                       : reinterpret_cast<const int *>(c.q);
                perm_v[u] = *pp;
            }
            // codebook operand of LUT tile t (B of the MFMA below): lane l
            // holds centroid ct*16 + l%16 of block bg*4 + l/16, hi and lo,
            // stored in lane order (1 KB contiguous per load); tiles past
            // the last centroid reload the last tile
            const int nct = (c.n_centroids + 15) / 16;
#pragma unroll
            for (int t = 0; t < LT; ++t) {
                const int flat = wv * LT + t, bg = flat / 16, ct = min(flat % 16, nct - 1);
                const uint4 *cp = c.codebook + (bg * nct + ct) * 2 * kWave + lane;
                cb_hi[t] = cp[0];
                cb_lo[t] = cp[kWave];
            }
        }
        if constexpr (kShPre && K::kShareLdsTok > 0) {
            if (sh_lds) {
                // 16 bytes a lane: copy i of the share's rows covers rows
                // (i*64 + lane) / (D/8), keys for i < n_copies, then values
                constexpr int CPR = D / 8;  // 16-byte chunks per row
                const int64_t head = bb * va.buf_sb + kvh * va.buf_sh;
                const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(sh_k));
                const int n_copies = (n_sh * CPR + kWave - 1) / kWave;
                for (int i = 0; wv == 0 && i < 2 * n_copies; ++i) {  // wave 0, which attends it
                    const bool is_v = i >= n_copies;
                    const int ci = (is_v ? i - n_copies : i) * kWave + lane;
                    const int row = min(ci / CPR, n_sh - 1), chunk = ci % CPR;
                    const char *src = static_cast<const char *>(is_v ? va.vbuf : va.kbuf) +
                                      ((head + (bj0 + row) * va.buf_st) * 2 + chunk * 16);
                    if constexpr (kHStep) src = ex_row(va, is_v, bj0 + row) + chunk * 16;
                    const uint32_t dst = lds0 + (uint32_t)((is_v ? K::kShareLdsTok * D * 2 : 0) +
                                                           (is_v ? i - n_copies : i) * 1024);
                    __builtin_amdgcn_global_load_lds(src, reinterpret_cast<lds_t<void> *>(dst), 16, 0, 0);
                }
            }
        }
        if constexpr (kShPre) {
            if (sh_pre) {
                const unsigned short *kb = static_cast<const unsigned short *>(va.kbuf);
                const unsigned short *vb = static_cast<const unsigned short *>(va.vbuf);
                const int64_t head = bb * va.buf_sb + kvh * va.buf_sh;
#pragma unroll
                for (int j = 0; j < NSH; ++j) {
                    const int64_t jt = bj0 + min(j, n_sh - 1);
                    const unsigned short *kr = kb + head + jt * va.buf_st;
                    const unsigned short *vr = vb + head + jt * va.buf_st;
                    if constexpr (kHStep) {
                        kr = reinterpret_cast<const unsigned short *>(ex_row(va, false, jt));
                        vr = reinterpret_cast<const unsigned short *>(ex_row(va, true, jt));
                    }
#pragma unroll
                    for (int k = 0; k < DLh; ++k) {
                        hk_raw[j][k] = kr[lane + kWave * k];
                        hv_raw[j][k] = vr[lane + kWave * k];
                    }
                }
            }
        }
        // A fused step's last split: the new tokens' key and value rows
        // (lane: dims lane + 64k), the permutation entries of the key dims
        // its A lanes hold and its centroids' norms load here, before the
        // loader streams anything, so none of them waits behind its tiles
        // (a hybrid step: the flushed tokens' rows, the code words their
        // codes go into, and the new tokens that go into the buffer)
        int pk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        float nrm[kStep ? LT : 1];
        using PutT = std::conditional_t<D == 128, uint32_t, unsigned short>;  // a lane's dims of a row
        static_assert(D == 128 || D == 64, "head_dim");
        PutT kput_r[kHStep ? NS : 1], vput_r[kHStep ? NS : 1];
        uint32_t cw_pre[2][DLs];
        const bool put_wave = kHStep && split == c.n_splits - 1 && rg == 0 && wv == NC - 1;
        const bool code_wave = kHStep && n_step > 0 && rg == 0 && wv == (NC > 1 ? 1 : 0);
        if constexpr (kHStep) {
            if (put_wave) {
                const int n_new = (int)(va.t_buf - va.n_rem);  // >= 1 (checked on the host)
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    const int ii = min(i, n_new - 1);
                    kput_r[i] = reinterpret_cast<const PutT *>(ex_row(va, false, va.n_rem + ii))[lane];
                    vput_r[i] = reinterpret_cast<const PutT *>(ex_row(va, true, va.n_rem + ii))[lane];
                }
            }
            if constexpr (VF::kStepQuant) {
            if (code_wave) {
                constexpr int TPW = 32 / VF::kBits;
                const int64_t w0 = c.t_kv / TPW, wmax = c.cap / TPW - 1;
#pragma unroll
                for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
                    for (int k = 0; k < DLs; ++k)
                        cw_pre[s2][k] = va.codes_out[(bh * (c.cap / TPW) + min(w0 + s2, wmax)) * D +
                                                     lane + kWave * k];
            }
            }
        }
        if constexpr (kStep) {
            if (n_step > 0) {
                // (float16 tokens, checked on the host: plain 2-byte loads,
                // all in flight together)
                const int64_t head = bb * va.buf_sb + kvh * va.buf_sh;
                const __half *kh = static_cast<const __half *>(va.kbuf);
                const __half *vh = static_cast<const __half *>(va.vbuf);
                __half kraw[NS][DLs], vraw[NS][DLs];
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int k = 0; k < DLs; ++k) {
                        const int64_t o = head + (int64_t)min(j, n_step - 1) * va.buf_st + lane + kWave * k;
                        kraw[j][k] = kh[o];
                        vraw[j][k] = vh[o];
                    }
#pragma unroll
                for (int j = 0; j < NS; ++j)
#pragma unroll
                    for (int k = 0; k < DLs; ++k) {
                        kpre[j][k] = __half2float(kraw[j][k]);
                        vpre[j][k] = __half2float(vraw[j][k]);
                    }
                // lane l of the key products holds K slice l/16 (block
                // (wv*LT/16)*4 + l/16) of row l%16
                const int kb = ((wv * LT) / 16) * 4 + g;
#pragma unroll
                for (int i = 0; i < 8; ++i) pk[i] = c.perm ? c.perm[kb * 8 + i] : kb * 8 + i;
                // (the prepared tiles' order; tiles past the last centroid
                // reread the last one, as the LUT build's loads)
                const int nct = (c.n_centroids + 15) / 16;
#pragma unroll
                for (int t = 0; t < LT; ++t) {
                    const int flat = wv * LT + t;
                    nrm[t] = va.cb_norms[((flat / 16) * nct + min(flat % 16, nct - 1)) * kWave + lane];
                }
            }
        }
        // (after a step's loads, which the step's encode waits on before the
        // unit is needed)
        if constexpr (kRegs) {
            // this wave's first unit streams into registers while the LUT is built
            const int u0 = unit_of(0);
            if (u0 < n_units) load_ru(ua, u0);
        } else if constexpr (K::kPriv) {
            // this wave's first units (u = wv + k*NC) stream in while the LUT is built
            for (; nq < K::kPrivSlots && wv + nq * NC < n_units; ++nq)
                issue_at(wv + nq * NC, ring_l + priv_slot(nq));
        }
        lds_barrier();  // small loads issued, flags initialised
        // query elements: round_to(q_dtype, q * scale) (attention.py:208)
#pragma unroll
        for (int u = 0; u < QE; ++u) {
            const int e = tid + u * CT, er = e / D;
            if (e < R * D) {
                float qv = 0.f;
                if (row_ok(er)) {
                    const uint32_t w = q_word[u];
                    const uint32_t h = (q_byte[u] & 2) ? (w >> 16) : (w & 0xffffu);
                    if (c.q_dtype == SS_F32)
                        qv = __uint_as_float(w);
                    else if (c.q_dtype == SS_F16)
                        qv = __half2float(__ushort_as_half((unsigned short)h));
                    else
                        qv = __uint_as_float(h << 16);
                }
                qraw[e] = round_to(c.q_dtype, qv * c.scale);
                if (has_ex) bpart[2 * R + e] = qraw[e];
            }
        }
        compute_barrier(1);  // raw query staged
        // codec permutation of the query dims (attention.py:228)
#pragma unroll
        for (int u = 0; u < QE; ++u) {
            const int e = tid + u * CT, er = e / D, ej = e - (e / D) * D;
            if (e < R * D) {
                const int src = c.perm ? min(max(perm_v[u], 0), D - 1) : ej;
                qp[e] = qraw[er * D + src];
            }
        }
        compute_barrier(2);
        // Non-fp16 queries enter the split-fp16 products scaled per row by the
        // power of two 2^-s_r that brings row r's largest element into
        // [2^14, 2^15), so their fp16 hi parts never overflow whatever the
        // query's magnitude; the products are multiplied back by 2^s_r.
        f32x4 qsc = f32x4{1.f, 1.f, 1.f, 1.f};  // 2^s_r of rows 0..3
        float qinv = 1.f;                         // 2^-s of query row lane & 3
        if (c.q_dtype != SS_F16) {
            static_assert(R == 4, "four query rows per column");
            float mx = 0.f;
            for (int j = l16; j < D; j += 16) mx = fmaxf(mx, fabsf(qp[g * D + j]));
#pragma unroll
            for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
            const int sh = row_exp_shift(mx);  // row g's shift, lanes 16g .. 16g+15
            qsc = f32x4{exp2i(__shfl(sh, 0)), exp2i(__shfl(sh, 16)), exp2i(__shfl(sh, 32)),
                        exp2i(__shfl(sh, 48))};
            qinv = exp2i(-__shfl(sh, 16 * (lane & 3)));
        }
        {
            // LUT entry (b, cc) holds the 4 rows' dot products, in log2 units,
            // computed on the matrix cores: for 4 blocks bg*4+s and 16
            // centroids at once, D[4s + r][n] = sum_k A[4s + r][k] B[k][n]
            // with K = 32 = 4 blocks x 8 dims, A block-diagonal (row 4s + r
            // holds query row r's dims of block s in the K slice of block s,
            // zero elsewhere) and B[k][n] the dims of centroid n.  Operands
            // are split fp16: x = hi + lo * 2^-11 for the codebook (prepared
            // with a power-of-two scale) and, unless the query is already
            // fp16, for the query; products of fp16 parts are exact and
            // accumulate in fp32.
            const int bg = (wv * LT) / 16;
            const int ar = l16 & 3;                  // query row of this A lane
            const bool a_live = (l16 >> 2) == g;     // block-diagonal
            const lds_t<f32x4> *qp4 = to_lds<f32x4>(qp);
            const f32x4 x0 = qp4[(ar * D + (bg * 4 + g) * kBlockDim) / 4];
            const f32x4 x1 = qp4[(ar * D + (bg * 4 + g) * kBlockDim) / 4 + 1];
            const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            f16x8 a_hi, a_lo;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x = a_live ? xs[i] * qinv : 0.f;
                const _Float16 h = (_Float16)x;
                a_hi[i] = h;
                a_lo[i] = (_Float16)((x - (float)h) * kSplitScale);
            }
            const float mul = cb_mul * kLog2e;
            const float mul_lo = mul * (1.f / kSplitScale);
            // all products first (back to back on the matrix core), then
            // scale and store; tiles past the last centroid are computed on
            // the reloaded last tile and not stored
            auto build = [&](auto q_split) {
                constexpr int G = 4;  // tiles per group: products of group k+1 overlap stores of k
                static_assert(LT % G == 0, "LUT tile groups");
                f32x4 hh[G], cr[G];
                auto products = [&](int t0) {
#pragma unroll
                    for (int u = 0; u < G; ++u) {
                        const f16x8 bh = __builtin_bit_cast(f16x8, cb_hi[t0 + u]);
                        const f16x8 bl = __builtin_bit_cast(f16x8, cb_lo[t0 + u]);
                        const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
                        hh[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, bh, z, 0, 0, 0);
                        cr[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi, bl, z, 0, 0, 0);
                        if constexpr (decltype(q_split)::value)
                            cr[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo, bh, cr[u], 0, 0, 0);
                    }
                };
#pragma unroll
                for (int t0 = 0; t0 < LT; t0 += G) {
                    products(t0);
#pragma unroll
                    for (int u = 0; u < G; ++u) {
                        f32x4 e = hh[u] * mul + cr[u] * mul_lo;
                        if constexpr (decltype(q_split)::value) e *= qsc;
                        const int cc = ((wv * LT + t0 + u) % 16) * 16 + l16;
                        if (cc < c.n_centroids)
                            lut4[(bg * 4 + g) * kLutStride + cc] = make_float4(e.x, e.y, e.z, e.w);
                    }
                }
            };
            // fp16 queries have lo == 0
            if (c.q_dtype == SS_F16)
                build(std::false_type{});
            else
                build(std::true_type{});
        }
        // a fused step's new keys, this lane's block (token l%4's dims in A
        // lanes), and |k|^2 of its block for the four tokens
        float kd[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        float kkr[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (kStep) {
            if (n_step > 0) {
                // The new tokens' keys encoded from the codebook operands
                // this wave holds for the LUT (its 4 blocks x 256 centroids):
                // the key . centroid products on the matrix cores (token r of
                // block bg*4 + s in A row 4s + r, fp16 keys exact), then
                // D'(c) = |k|^2 + |C_c|^2 - 2 k . C_c in float32, |C_c|^2 from
                // the prepared codebook.  The prepared centroids hold 22 bits
                // (|C - C'| <= 2^-22 |C| per element, plus a floor under 2^-45
                // of the largest), so |D' - D| <= E = 2^-20 (|k| + max|C|)^2 +
                // 2^-31 m |k| (m the codebook's power-of-two scale, the
                // product and sum roundings included): when the runner-up
                // clears the best by 2E the best is the exact nearest centroid;
                // otherwise the block is ranked exactly (the encoder's
                // exact_block_wave over the float32 centroids).
                const int bg = (wv * LT) / 16;
                const int ar = l16 & 3;
                const bool a_row = (l16 >> 2) == g;
#pragma unroll
                for (int j = 0; j < NS; ++j) {
                    if (j < n_step) {
#pragma unroll
                        for (int i = 0; i < 8; ++i) {
                            const int p = min(max(pk[i], 0), D - 1);
                            const float x0 = __shfl(kpre[j][0], p & (kWave - 1));
                            const float x1 = __shfl(kpre[j][DLs - 1], p & (kWave - 1));
                            kd[i] = ar == j ? ((p >> 6) ? x1 : x0) : kd[i];
                        }
                    }
                }
                f16x8 ak;
                float kk = 0.f;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const bool live = a_row && ar < n_step;
                    ak[i] = live ? (_Float16)kd[i] : (_Float16)0.f;
                    kk = fmaf(kd[i], kd[i], kk);
                }
                // |k|^2 of (this lane's block g, token r) sits in lane 20g + r
#pragma unroll
                for (int r = 0; r < 4; ++r) kkr[r] = __shfl(kk, 20 * g + r);
                const float m2 = -2.f * cb_mul;
                float best[4], second[4], nmax = 0.f;
                int bidx[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    best[r] = INFINITY;
                    second[r] = INFINITY;
                    bidx[r] = 0x7fffffff;
                }
                const int nct_ = (c.n_centroids + 15) / 16;
#pragma unroll
                for (int t = 0; t < LT; ++t) {
                    const f32x4 z = f32x4{0.f, 0.f, 0.f, 0.f};
                    const f32x4 dh = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        ak, __builtin_bit_cast(f16x8, cb_hi[t]), z, 0, 0, 0);
                    const f32x4 dl = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                        ak, __builtin_bit_cast(f16x8, cb_lo[t]), z, 0, 0, 0);
                    const int ct = (wv * LT + t) % 16;
                    const int cc = ct * 16 + l16;
                    if (ct < nct_ && cc < c.n_centroids) {
                        nmax = fmaxf(nmax, nrm[t]);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float dot = dh[r] + dl[r] * (1.f / kSplitScale);
                            const float dd = fmaf(m2, dot, kkr[r] + nrm[t]);
                            const bool lt = dd < best[r];
                            second[r] = lt ? best[r] : fminf(second[r], dd);
                            bidx[r] = lt ? cc : bidx[r];
                            best[r] = lt ? dd : best[r];
                        }
                    }
                }
                // the 16 lanes of each block: (best, runner-up, index), the
                // largest norm
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    nmax = fmaxf(nmax, __shfl_xor(nmax, o));
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float ob = __shfl_xor(best[r], o), os = __shfl_xor(second[r], o);
                        const int oi = __shfl_xor(bidx[r], o);
                        const bool mine = best[r] < ob || (best[r] == ob && bidx[r] < oi);
                        second[r] = mine ? fminf(second[r], ob) : fminf(os, best[r]);
                        best[r] = mine ? best[r] : ob;
                        bidx[r] = mine ? bidx[r] : oi;
                    }
                }
                // this wave's candidates: (best, runner-up, index, largest
                // norm) per (block, token), merged below with the waves that
                // hold the group's other centroid tiles (head_dim 64)
                if (l16 == 0) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        step_part[(wv * 4 + g) * 4 + r] =
                            f32x4{best[r], second[r], __int_as_float(bidx[r]), nmax};
                }
            }
        }
        // fp16 heavy-block key dims (mixed-precision codecs; their LUT
        // entries are zero): A operands of v_mfma_f32_4x4x4f16 products with
        // each token's own dims, query row lane%4, dims 4kk .. 4kk+3, split
        // fp16 hi and lo * 2^11 (the lo part only for non-fp16 queries)
        constexpr int HK = HV ? kMaxHeavyMfma / 4 : 1;
        f16x4 hah[HK], hal[HK];
        const int nh4 = HV ? c.nhd >> 2 : 0;
        if constexpr (HV) {
#pragma unroll
            for (int kk = 0; kk < HK; ++kk) {
                hah[kk] = hal[kk] = f16x4{};
                if (kk < nh4) {
#pragma unroll
                    for (int e2 = 0; e2 < 4; ++e2) {
                        const int hd = min(max(c.heavy_dims[4 * kk + e2], 0), D - 1);
                        const float x = qp[(lane & 3) * D + hd] * qinv;
                        const _Float16 h = (_Float16)x;
                        hah[kk][e2] = h;
                        hal[kk][e2] = (_Float16)((x - (float)h) * kSplitScale);
                    }
                }
            }
        }
        compute_barrier(3);  // LUT complete (the query in LDS is read for the last time)
        if constexpr (kStep) {
            if (n_step > 0) {
                // the first wave of each block group merges the group's
                // waves' candidates (16 / LT of them) and decides
                constexpr int WPG = 16 / LT;  // waves per 4-block group
                if ((wv * LT) % 16 == 0) {
                    const int bg = (wv * LT) / 16;
                    uint32_t need = 0u;
                    if (l16 == 0) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            if (r < n_step) {
                                f32x4 a = step_part[(wv * 4 + g) * 4 + r];
#pragma unroll
                                for (int w2 = 1; w2 < WPG; ++w2) {
                                    const f32x4 o = step_part[((wv + w2) * 4 + g) * 4 + r];
                                    const int ai = __float_as_int(a[2]), oi = __float_as_int(o[2]);
                                    const bool mine = a[0] < o[0] || (a[0] == o[0] && ai < oi);
                                    const float sec = mine ? fminf(a[1], o[0]) : fminf(o[1], a[0]);
                                    a = mine ? f32x4{a[0], sec, a[2], fmaxf(a[3], o[3])}
                                             : f32x4{o[0], sec, o[2], fmaxf(a[3], o[3])};
                                }
                                const float kn = __builtin_sqrtf(kkr[r]);
                                const float a2 = kn + __builtin_sqrtf(a[3]);
                                const float e = fmaf(0x1p-20f * a2, a2, 0x1p-31f * cb_mul * kn);
                                const int bi = __float_as_int(a[2]);
                                const bool ok = a[1] - a[0] > 2.f * e && bi != 0x7fffffff;
                                if (ok) {
                                    step_idx[r * NB + bg * 4 + g] = (uint8_t)bi;
                                    if (kHStep && rg == 0)
                                        va.idx_out[(bh * c.cap + c.t_kv + r) * NB + bg * 4 + g] = (uint8_t)bi;
                                }
                                need |= ok ? 0u : (1u << r);
                            }
                        }
                    }
                    // exact ranking for the pairs not cleared (rare): the whole
                    // wave over the float32 centroids, one pair at a time (one
                    // copy of the code, entered only when some pair needs it:
                    // unrolled, its sixteen inlined copies cost instruction
                    // fetches on every step)
                    if (__builtin_amdgcn_ballot_w64(need != 0u) != 0) {
#pragma unroll 1
                    for (int s2 = 0; s2 < 4; ++s2) {
#pragma unroll 1
                        for (int r = 0; r < 4; ++r) {
                            const bool any =
                                __builtin_amdgcn_ballot_w64(g == s2 && ((need >> r) & 1u)) != 0;
                            if (any) {
                                float kv[8];
#pragma unroll
                                for (int i = 0; i < 8; ++i) kv[i] = __shfl(kd[i], 20 * s2 + r);
                                const int b = bg * 4 + s2;
                                const int bi = exact_block_wave<8>(
                                    kv, va.centroids + (int64_t)b * c.n_centroids * 8, c.n_centroids, lane);
                                if (lane == 0) {
                                    step_idx[r * NB + b] = (uint8_t)bi;
                                    if (kHStep && rg == 0)
                                        va.idx_out[(bh * c.cap + c.t_kv + r) * NB + b] = (uint8_t)bi;
                                }
                            }
                        }
                    }
                    }
                    if constexpr (kHStep) {
                        // this group's indices are in LDS (and stored): tell
                        // wave 0, which scores the flushed tokens; the other
                        // waves go on to their units
                        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                        if (lane == 0)
                            __hip_atomic_fetch_add(const_cast<lds_t<int> *>(cbar + 2), 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
                    }
                }
                if constexpr (kStepOnly) compute_barrier(4);  // the new tokens' index rows are complete
                if (kStepOnly && rg == 0) {
                    // the cache's copy at positions t_kv .. t_kv + n_new - 1:
                    // index rows, then (wave 0's lanes) the fp16 values
                    for (int e = wv * kWave + lane; e < n_step * NB; e += NC * kWave)
                        va.idx_out[(bh * c.cap + c.t_kv + e / NB) * NB + e % NB] = step_idx[e];
                    if constexpr (kStepOnly) {
                        if (wv == 0) {
#pragma unroll
                            for (int j = 0; j < NS; ++j)
                                if (j < n_step)
#pragma unroll
                                    for (int k = 0; k < DLs; ++k)
                                        store_value_il8(va.v8_out, bh, c.cap, D, c.t_kv + j,
                                                        lane + kWave * k, vpre[j][k]);
                        }
                    }
                }
                if constexpr (kHStep && !StepQuantOf<VF>::value) {
                    if (code_wave) {
                        // the flushed tokens' fp16 values into the interleaved values
#pragma unroll
                        for (int j = 0; j < NS; ++j)
                            if (j < n_step)
#pragma unroll
                                for (int k = 0; k < DLs; ++k)
                                    store_value_il8(va.v8_out, bh, c.cap, D, c.t_kv + j, lane + kWave * k,
                                                    vpre[j][k]);
                    }
                }
                if constexpr (StepQuantOf<VF>::value) {
                    if (code_wave) {
                        // the flushed tokens' codes into their words (the
                        // other tokens' bits kept: token i of a word at bit
                        // bits*(i/2) + 16*(i%2)), and each group's scale and
                        // zero from the lane holding its first dim
                        using SZT = typename VF::SzT;
                        constexpr int TPW = 32 / VF::kBits;
                        constexpr uint32_t cmask = (1u << VF::kBits) - 1u;
                        constexpr int G = D / VF::kNG;
                        const int64_t w0 = c.t_kv / TPW;
                        const int64_t cw_head = bh * (c.cap / TPW);
                        uint32_t wa0[DLs], wa1[DLs];
#pragma unroll
                        for (int k = 0; k < DLs; ++k) {
                            wa0[k] = cw_pre[0][k];
                            wa1[k] = cw_pre[1][k];
                        }
#pragma unroll
                        for (int j = 0; j < NS; ++j) {
                            if (j < n_step) {
                                float qc[DLs], qs[DLs], qz[DLs];
                                quantize_token_wave<D, VF::kBits, VF::kNG>(vpre[j], qc, qs, qz);
                                const int64_t t = c.t_kv + j;
                                const bool second = t / TPW != w0;
                                const int i = (int)(t % TPW);
                                const int pos = VF::kBits * (i >> 1) + 16 * (i & 1);
#pragma unroll
                                for (int k = 0; k < DLs; ++k) {
                                    const uint32_t cv = ((uint32_t)qc[k] & cmask) << pos;
                                    if (second)
                                        wa1[k] = (wa1[k] & ~(cmask << pos)) | cv;
                                    else
                                        wa0[k] = (wa0[k] & ~(cmask << pos)) | cv;
                                    const int d = lane + kWave * k;
                                    if (d % G == 0) {
                                        const int64_t srow = (bh * c.cap + t) * VF::kNG + d / G;
                                        va.scales_out[srow] = (SZT)qs[k];
                                        va.zeros_out[srow] = (SZT)qz[k];
                                    }
                                }
                            }
                        }
                        const bool two = (c.t_kv + n_step - 1) / TPW != w0;
#pragma unroll
                        for (int k = 0; k < DLs; ++k) {
                            va.codes_out[(cw_head + w0) * D + lane + kWave * k] = wa0[k];
                            if (two) va.codes_out[(cw_head + w0 + 1) * D + lane + kWave * k] = wa1[k];
                        }
                    }
                }
            }
        }
        if constexpr (kHStep) {
            if (put_wave) {
                // the step's new tokens into the buffer rows after the window
                const int n_new = (int)(va.t_buf - va.n_rem);
                const int64_t row0 = va.n_flush + va.n_rem;
#pragma unroll
                for (int i = 0; i < NS; ++i) {
                    if (i < n_new) {
                        const int64_t o = (bb * va.buf_sb + kvh * va.buf_sh + (row0 + i) * va.buf_st) * 2;
                        reinterpret_cast<PutT *>(static_cast<char *>(va.kput) + o)[lane] = kput_r[i];
                        reinterpret_cast<PutT *>(static_cast<char *>(va.vput) + o)[lane] = vput_r[i];
                    }
                }
            }
        }
        if constexpr (VF::kHybridBuffer)
            if (wv == 0 && has_buf) buffer_share(va);

        _Float16 *pw = pst + wv * VF::kPRows * kPStride;
        // one 64-token unit of this wave: scores, online softmax, P.V
        auto step = [&](const IdxRow<NB> &ir, typename VF::Tile &tv, const uint4 (&khv)[HVN],
                        int u) __attribute__((always_inline)) {
            const int64_t t0 = t_beg + (int64_t)u * kWave;
            // tokens of this tile still inside the split (wave-uniform, 1..64)
            const int n_in = (int)min(t_end - t0, (int64_t)kWave);
            // scores from the LUT: every block's read in flight at once, then
            // a tree sum (one LDS round trip)
            f32x4 e[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) e[b] = lut_l[b * kLutStride + ir.at(b)];
#pragma unroll
            for (int w = 1; w < NB; w *= 2)
#pragma unroll
                for (int b = 0; b < NB; b += 2 * w) e[b] += e[b + w];
            float sc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) sc[r] = e[0][r];
            if constexpr (HV) {
                if (nh4 > 0) {  // heavy dims on the matrix cores: D[row][token lane]
                    f32x4 hs = f32x4{0.f, 0.f, 0.f, 0.f}, hl = hs;
#pragma unroll
                    for (int j8 = 0; j8 < kMaxHeavyMfma / 8; ++j8)
                        if (2 * j8 < nh4) {
                            const f16x4 b0 = __builtin_bit_cast(f16x4, make_uint2(khv[j8].x, khv[j8].y));
                            const f16x4 b1 = __builtin_bit_cast(f16x4, make_uint2(khv[j8].z, khv[j8].w));
                            hs = __builtin_amdgcn_mfma_f32_4x4x4f16(hah[2 * j8], b0, hs, 0, 0, 0);
                            hs = __builtin_amdgcn_mfma_f32_4x4x4f16(hah[2 * j8 + 1], b1, hs, 0, 0, 0);
                        }
                    if (c.q_dtype != SS_F16) {
#pragma unroll
                        for (int j8 = 0; j8 < kMaxHeavyMfma / 8; ++j8)
                            if (2 * j8 < nh4) {
                                const f16x4 b0 = __builtin_bit_cast(f16x4, make_uint2(khv[j8].x, khv[j8].y));
                                const f16x4 b1 = __builtin_bit_cast(f16x4, make_uint2(khv[j8].z, khv[j8].w));
                                hl = __builtin_amdgcn_mfma_f32_4x4x4f16(hal[2 * j8], b0, hl, 0, 0, 0);
                                hl = __builtin_amdgcn_mfma_f32_4x4x4f16(hal[2 * j8 + 1], b1, hl, 0, 0, 0);
                            }
                    }
                    const f32x4 hv = (hs + hl * (1.f / kSplitScale)) * (qsc * kLog2e);
#pragma unroll
                    for (int r = 0; r < R; ++r) sc[r] += hv[r];
                }
            }
            // A whole tile every row sees (no causal cut, no split end) whose
            // scores all stay at most kLag above the rows' running maxima
            // keeps the maxima: no reduction, no rescale (its probabilities
            // are at most 2^kLag; l and acc stay relative to the same
            // maxima).  Otherwise masked lanes add -inf (their index rows are
            // real, clamped tokens, so the sums are finite) and the maxima
            // are reduced over the wave.
            bool moved = true;
            if (n_in == kWave && t0 + (kWave - 1) <= lim_min) {
                uint64_t above = 0;
#pragma unroll
                for (int r = 0; r < R; ++r) above |= __builtin_amdgcn_ballot_w64(sc[r] > m[r] + kLag);
                moved = above != 0;
            } else {
                const bool kok = lane < n_in;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    // last visible lane of row r (causal), wave-uniform
                    const int lim_rel = (int)max(min(lim[r] - t0, (int64_t)kWave), (int64_t)-1);
                    sc[r] += (kok && lane <= lim_rel) ? 0.f : -INFINITY;
                }
            }
            float corr[R], p[R];
            if (moved) {
                float tmax[R];
                wave_max4_dpp(sc, tmax);  // the four rows' reductions interleaved
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const float mn = fmaxf(m[r], tmax[r]);
                    corr[r] = fast_exp2(m[r] - mn);
                    p[r] = fast_exp2(sc[r] - mn);
                    lsum[r] = fmaf(lsum[r], corr[r], p[r]);
                    m[r] = mn;
                }
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    corr[r] = 1.f;
                    p[r] = fast_exp2(sc[r] - m[r]);
                    lsum[r] += p[r];
                }
            }
            VF::pv(tv, vst, acc, p, corr, moved, n_in, pw, lane);
        };
        if constexpr (kRegs) {
            // two register sets in turn (past the last unit the loads repeat
            // the last one, so the loop stays straight-line)
            for (int i = 0, u = unit_of(0); u < n_units;) {
                const int u1 = unit_of(++i);
                load_ru(ub, min(u1, n_units - 1));
                {
                    typename VF::Tile tv;
                    VF::from_raw(tv, ua.raw, lane);
                    step(ua.ir, tv, ua.khv, u);
                }
                if (u1 >= n_units) break;
                const int u2 = unit_of(++i);
                load_ru(ua, min(u2, n_units - 1));
                {
                    typename VF::Tile tv;
                    VF::from_raw(tv, ub.raw, lane);
                    step(ub.ir, tv, ub.khv, u1);
                }
                u = u2;
            }
        } else {
        for (int u = wv, uk = 0; u < n_units; u += NC, ++uk) {
            const int j = u / K::kSub, sub = u - j * K::kSub;  // ring tile, sub-tile
            const int slot = K::kPriv ? uk % K::kPrivSlots : j % K::kSlots;
            // the heavy dims of token `lane` (the split's last token past its
            // end), loaded while the tile is waited on and the LUT read
            uint4 khv[HVN];
            if constexpr (HV) {
                if (nh4 > 0) {
                    const int64_t tk = min(t_beg + (int64_t)u * kWave + lane, t_last);
                    const uint4 *hp = reinterpret_cast<const uint4 *>(c.kheavy + (bh * c.cap + tk) * c.nhd);
#pragma unroll
                    for (int j8 = 0; j8 < kMaxHeavyMfma / 8; ++j8)
                        if (2 * j8 < nh4) khv[j8] = hp[j8];
                }
            }
            if constexpr (K::kPriv) {
                // this wave's copies of unit u have landed (its later units
                // stay in flight)
                wait_oldest_tile<LPT, K::kPrivSlots>(nq - uk);
            } else {
                int spins = 0;
                while (ready[slot] != j) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > c.spin_limit) {
                        wait_gave_up(kWaitTile);
                        break;
                    }
                }
            }
            asm volatile("" ::: "memory");
            // copy the tile (index rows and values) into registers and
            // release the slot at once
            const char *sb = K::kPriv ? ring + priv_slot(slot) : ring + slot * K::kSlot;
            const char *ib = sb + K::kTileV + sub * K::kTileI1;
            IdxRow<NB> ir;
            if constexpr (NB == 16) {
                const uint4 w4 = *reinterpret_cast<const uint4 *>(ib + lane * 16);
                ir.w[0] = w4.x; ir.w[1] = w4.y; ir.w[2] = w4.z; ir.w[3] = w4.w;
            } else {
                const uint2 w2 = *reinterpret_cast<const uint2 *>(ib + lane * 8);
                ir.w[0] = w2.x; ir.w[1] = w2.y;
            }
            typename VF::Tile tv;
            VF::copy(tv, sb, sub, lane);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if constexpr (K::kPriv) {
                // the slot's data is in registers: refill it with this wave's next unit
                if (wv + nq * NC < n_units) {
                    issue_at(wv + nq * NC, ring_l + priv_slot(nq % K::kPrivSlots));
                    ++nq;
                }
            } else {
                if (lane == 0) done[slot * K::kSub + sub] = j;
            }
            step(ir, tv, khv, u);
        }
        }
    }
    __syncthreads();  // every tile consumed; the ring is free for the merge

    // wave results: the value format hands each wave's accumulators to LDS
    // as (hi, lo) parts (wa[w][0 = hi, 1 = lo][r][d]) and the combine adds
    // them, so every read of the combine can be issued at once (one LDS
    // round trip)
    float *wm = reinterpret_cast<float *>(ring);
    float *wl = wm + NC * R;
    float *wa = wl + NC * R;  // [NC][2][R][D]
    static_assert((2 * NC * R) % 4 == 0, "wa alignment");
    if (!loader) {
        {
            float ls[R];
            wave_sum4_dpp(lsum, ls);
#pragma unroll
            for (int r = 0; r < R; ++r) lsum[r] = ls[r];
        }
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wm[wv * R + r] = m[r];
                wl[wv * R + r] = lsum[r];
            }
        }
        if constexpr (VfArgsToLds<VF>::value)
            VF::to_lds_args(acc, vst, va, wa + wv * 2 * R * D, lane);
        else
            VF::to_lds(acc, vst, wa + wv * 2 * R * D, lane);
    }
    __syncthreads();
    // combine the compute waves' (m, l, acc) of row r into this workgroup's
    // (M, L, A) for dims d0 .. d0+3
    const lds_t<f32x4> *wa4 = to_lds<f32x4>(wa);
    auto combine4 = [&](int r, int d0, float &M, float &L, f32x4 &A) {
        float mw[NC], lw[NC];
        f32x4 hi[NC], lo[NC];
#pragma unroll
        for (int w = 0; w < NC; ++w) {
            mw[w] = wm[w * R + r];
            lw[w] = wl[w * R + r];
            hi[w] = wa4[(((w * 2 + 0) * R + r) * D + d0) / 4];
            lo[w] = wa4[(((w * 2 + 1) * R + r) * D + d0) / 4];
        }
        M = -1e30f;
#pragma unroll
        for (int w = 0; w < NC; ++w) M = fmaxf(M, mw[w]);
        float mb = -1e30f, lb = 0.f;
        f32x4 ab = f32x4{0.f, 0.f, 0.f, 0.f};
        if (has_buf) {  // the split's share of the token buffer
            mb = bpart[r];
            lb = bpart[R + r];
            ab = *reinterpret_cast<const f32x4 *>(bpart + 2 * R + r * D + d0);
            M = fmaxf(M, mb);
        }
        L = 0.f;
        A = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < NC; ++w) {
            const float f = fast_exp2(mw[w] - M);
            L = fmaf(lw[w], f, L);
            A += (hi[w] + lo[w]) * f;
        }
        if (has_buf) {
            const float f = fast_exp2(mb - M);
            L = fmaf(lb, f, L);
            A += ab * f;
        }
    };
    // Output rows: stored as they are, or, with c.rot, staged in LDS (the
    // LUT's space, free after the tile loop) and stored as y @ rot once
    // every dim of the rows is there (rot_rows, called by every thread).
    float *yrows = reinterpret_cast<float *>(smem);  // [R][D]
    auto put4 = [&](int r, int d0, f32x4 y) {
        if (c.rot) {
            *reinterpret_cast<float4 *>(yrows + r * D + d0) = make_float4(y[0], y[1], y[2], y[3]);
        } else if (row_ok(r)) {
            store4_from_f32(c.out, c.out_dtype, row_off(r) + d0, y[0], y[1], y[2], y[3]);
        }
    };
    auto rot_rows = [&]() {
        if (!c.rot) return;
        __syncthreads();
        for (int i = tid; i < R * D; i += THREADS) {
            const int r = i / D, d = i - r * D;
            if (!row_ok(r)) continue;
            const float *yr = yrows + r * D;
            float a0 = 0.f, a1 = 0.f;
#pragma unroll 8
            for (int k = 0; k < D; k += 2) {
                a0 = fmaf(yr[k], c.rot[k * D + d], a0);
                a1 = fmaf(yr[k + 1], c.rot[(k + 1) * D + d], a1);
            }
            store_from_f32(c.out, c.out_dtype, row_off(r) + d, a0 + a1);
        }
    };
    const int S = c.n_splits;
    if (S == 1) {
        for (int i = tid; i < R * D / 4; i += THREADS) {
            const int r = i / (D / 4), d0 = (i - r * (D / 4)) * 4;
            float M, L;
            f32x4 A;
            combine4(r, d0, M, L, A);
            const float iv = L > 0.f ? 1.f / L : 0.f;
            put4(r, d0, A * iv);
        }
        rot_rows();
        return;
    }

    // Split-T finish inside the kernel.  Every split stores its partial with
    // sc1 (agent-coherent) buffer stores, which write through this XCD's L2,
    // waits until they have completed, then adds 1 to its column's counter
    // with an agent-scope atomic.  The split that sees S - 1 reads all the
    // column's partials with sc1 loads (never a stale L2 line) and writes
    // the merged rows; it also resets the counter for the next call.  No
    // workgroup waits for another, so nothing depends on scheduling order.
    const int n_cols = gridDim.y;
    const __amdgpu_buffer_rsrc_t acc_rs =
        raw_buffer(c.part_acc, (uint32_t)((int64_t)n_cols * S * R * D * 4));
    const __amdgpu_buffer_rsrc_t ml_rs = raw_buffer(c.part_ml, (uint32_t)((int64_t)n_cols * S * R * 8));
    const int64_t slot0 = ((int64_t)col * S + split) * R;
    for (int i = tid; i < R * D / 4; i += THREADS) {
        const int r = i / (D / 4), d0 = (i - r * (D / 4)) * 4;
        float M, L;
        f32x4 A;
        combine4(r, d0, M, L, A);
        __builtin_amdgcn_raw_buffer_store_b128(A, acc_rs, (uint32_t)(((slot0 + r) * D + d0) * 4), 0,
                                               kCpolSc1);
        if (d0 == 0)
            __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(M), __float_as_uint(L)}, ml_rs,
                                                  (uint32_t)((slot0 + r) * 8), 0, kCpolSc1);
    }
    if (!c.fused_merge) return;  // a merge launch follows
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
    __syncthreads();
    volatile lds_t<int> *last = cbar + 1;
    if (tid == 0)
        *last = __hip_atomic_fetch_add(c.part_cnt + (int64_t)col * c.cnt_stride, 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!*last) return;

    // Last split of this column: merge.  With up to kMergeParts *
    // kMergeLoads splits, thread (part, chunk) loads float4 `chunk` of the
    // partials of splits part, part + kMergeParts, ... and their (m, l) into
    // registers, every load in flight at once (one memory round trip; slots
    // past the last split reload it and get weight 0, so the loads stay
    // unconditional), weights them by its own maximum, and the parts
    // combine through LDS.
    constexpr int CH = R * D / 4;
    constexpr int kMergeParts = THREADS / CH >= 4 ? 4 : THREADS / CH;
    constexpr int kMergeLoads = kMergeParts >= 4 ? 8 : 16;
    if (kMergeParts >= 2 && S <= kMergeParts * kMergeLoads) {
        const int cidx = tid % CH, part = tid / CH;
        const int mr = cidx / (D / 4), md0 = (cidx - mr * (D / 4)) * 4;
        float Mr = -1e30f, Lr = 0.f;
        f32x4 Ar = f32x4{0.f, 0.f, 0.f, 0.f};
        if (part < kMergeParts) {
            f32x4 av[kMergeLoads];
            u32x2 mv[kMergeLoads];
#pragma unroll
            for (int j = 0; j < kMergeLoads; ++j) {
                const int s2 = min(part + kMergeParts * j, S - 1);
                const int64_t sl = ((int64_t)col * S + s2) * R + mr;
                av[j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      acc_rs, (uint32_t)((sl * D + md0) * 4), 0, kCpolSc1));
                mv[j] = __builtin_amdgcn_raw_buffer_load_b64(ml_rs, (uint32_t)(sl * 8), 0, kCpolSc1);
            }
#pragma unroll
            for (int j = 0; j < kMergeLoads; ++j)
                Mr = part + kMergeParts * j < S ? fmaxf(Mr, __uint_as_float(mv[j][0])) : Mr;
#pragma unroll
            for (int j = 0; j < kMergeLoads; ++j) {
                const float w = part + kMergeParts * j < S ? fast_exp2(__uint_as_float(mv[j][0]) - Mr) : 0.f;
                Lr = fmaf(__uint_as_float(mv[j][1]), w, Lr);
                Ar += av[j] * w;
            }
        }
        // parts 1.. hand their (M, L, A) to part 0 through LDS (the ring)
        float *pm = reinterpret_cast<float *>(ring);  // [kMergeParts - 1][6][CH]
        static_assert((kMergeParts - 1) * 6 * CH * 4 <= K::kRingBytes, "merge LDS");
        if (part >= 1 && part < kMergeParts) {
            float *q6 = pm + (part - 1) * 6 * CH;
            q6[cidx] = Mr;
            q6[CH + cidx] = Lr;
#pragma unroll
            for (int k = 0; k < 4; ++k) q6[(2 + k) * CH + cidx] = Ar[k];
        }
        __syncthreads();
        if (part == 0) {
#pragma unroll
            for (int p2 = 1; p2 < kMergeParts; ++p2) {
                const float *q6 = pm + (p2 - 1) * 6 * CH;
                const float m2 = q6[cidx], l2 = q6[CH + cidx];
                const f32x4 a2 = f32x4{q6[2 * CH + cidx], q6[3 * CH + cidx], q6[4 * CH + cidx],
                                       q6[5 * CH + cidx]};
                const float Mn = fmaxf(Mr, m2);
                const float fo = fast_exp2(Mr - Mn), fn = fast_exp2(m2 - Mn);
                Ar = Ar * fo + a2 * fn;
                Lr = Lr * fo + l2 * fn;
                Mr = Mn;
            }
            const float iv = Lr > 0.f ? 1.f / Lr : 0.f;
            put4(mr, md0, Ar * iv);
        }
        rot_rows();
        if (tid == 0)
            __hip_atomic_store(c.part_cnt + (int64_t)col * c.cnt_stride, 0, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // More splits: LDS (the ring) holds weights [S][R],
    // row sums [R], the splits' (m, l) [S][R], then a chunk of the partial
    // accumulators.  The (m, l) loads and the first chunk's copy are issued
    // together, so the merge costs one memory round trip per chunk.
    float *wts = reinterpret_cast<float *>(ring);  // [kMaxSplits][R]
    float *lrow = wts + kMaxSplits * R;            // [R] (+pad)
    u32x2 *mlb = reinterpret_cast<u32x2 *>(lrow + 64);
    const int chunk_off = ((kMaxSplits * R + 64) * 4 + S * R * 8 + 1023) & ~1023;
    char *chunk = ring + chunk_off;
    const int cs_max = (K::kRingBytes - chunk_off) / (R * D * 4);
    static_assert(((kMaxSplits * R + 64) * 4 + kMaxSplits * R * 8 + 1023) / 1024 * 1024 +
                          2 * R * D * 4 <= K::kRingBytes,
                  "merge LDS");
    static_assert((R * D * 4) % 1024 == 0, "merge chunk granularity");
    const uint32_t chunk_l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(chunk));
    // copy the partial accumulators of splits s0 .. s0+cs (contiguous) into LDS
    auto copy_chunk = [&](int s0, int cs) {
        const char *src = reinterpret_cast<const char *>(c.part_acc) +
                          (((int64_t)col * S + s0) * R) * D * 4;
        const int n_kb = cs * R * D * 4 / 1024;
        for (int kb = wv; kb < n_kb; kb += K::kWaves)
            __builtin_amdgcn_global_load_lds(src + kb * 1024 + lane * 16,
                                             reinterpret_cast<lds_t<void> *>(chunk_l + kb * 1024), 16,
                                             0, kCpolSc1);
    };
    u32x2 mlv[(kMaxSplits * R + THREADS - 1) / THREADS];
    constexpr int MLPT = (kMaxSplits * R + THREADS - 1) / THREADS;
#pragma unroll
    for (int k = 0; k < MLPT; ++k) {
        const int i2 = tid + k * THREADS;  // i2 = s * R + r
        if (i2 < S * R)
            mlv[k] = __builtin_amdgcn_raw_buffer_load_b64(
                ml_rs, (uint32_t)((((int64_t)col * S) * R + i2) * 8), 0, kCpolSc1);
    }
    copy_chunk(0, min(cs_max, S));
#pragma unroll
    for (int k = 0; k < MLPT; ++k) {
        const int i2 = tid + k * THREADS;
        if (i2 < S * R) mlb[i2] = mlv[k];
    }
    __syncthreads();
    if (wv < R) {  // wave r: weights exp2(m_s - M) and the merged l of row r
        const int r = wv;
        float M = -1e30f;
        for (int s2 = lane; s2 < S; s2 += kWave) M = fmaxf(M, __uint_as_float(mlb[s2 * R + r][0]));
        M = wave_max(M);
        float L = 0.f;
        for (int s2 = lane; s2 < S; s2 += kWave) {
            const u32x2 v = mlb[s2 * R + r];
            const float w = fast_exp2(__uint_as_float(v[0]) - M);
            wts[s2 * R + r] = w;
            L = fmaf(__uint_as_float(v[1]), w, L);
        }
        L = wave_sum(L);
        if (lane == 0) lrow[r] = L;
    }
    // thread i2 < R*D/4 accumulates dims 4*(i2 % (D/4)) .. +3 of row
    // i2 / (D/4) over the chunk's splits (float4 LDS reads, two accumulators)
    constexpr int CH4 = R * D / 4;
    static_assert(CH4 <= THREADS, "one float4 chunk per thread");
    const int mr = tid / (D / 4), md0 = (tid - (tid / (D / 4)) * (D / 4)) * 4;
    f32x4 acc0 = f32x4{0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
    for (int s0 = 0; s0 < S; s0 += cs_max) {
        const int cs = min(cs_max, S - s0);
        if (s0 > 0) {
            __syncthreads();  // previous chunk consumed
            copy_chunk(s0, cs);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // chunk landed; weights ready
        if (tid < CH4) {
            const lds_t<f32x4> *cf4 = to_lds<f32x4>(chunk);
            int s2 = 0;
#pragma unroll 4
            for (; s2 + 1 < cs; s2 += 2) {
                acc0 += cf4[((s2 * R + mr) * D + md0) / 4] * wts[(s0 + s2) * R + mr];
                acc1 += cf4[(((s2 + 1) * R + mr) * D + md0) / 4] * wts[(s0 + s2 + 1) * R + mr];
            }
            if (s2 < cs) acc0 += cf4[((s2 * R + mr) * D + md0) / 4] * wts[(s0 + s2) * R + mr];
        }
    }
    if (tid < CH4) {
        const float L = lrow[mr];
        const f32x4 A = acc0 + acc1;
        const float iv = L > 0.f ? 1.f / L : 0.f;
        put4(mr, md0, A * iv);
    }
    rot_rows();
    if (tid == 0)
        __hip_atomic_store(c.part_cnt + (int64_t)col * c.cnt_stride, 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// SunShape-value decode on the matrix cores: head_dim 128, value block_dim 4,
// at most 256 value centroids, four query rows per column.  Scores as in
// decode_attn_kernel (fp32 query x centroid LUT in LDS, built here on the
// vector ALUs, plus exact dot products over fp16 heavy-block key dims when
// NH8 > 0, NH8*8 of them).  P.V runs as O[row][dim] = sum_t P[row][t] V[t][dim]
// on v_mfma_f32_16x16x32_f16 with P entering as fp16 hi/lo rows of p * 2^11
// (rows 0-3 hi, 4-7 lo, as in VIl8) and V gathered from the value codebook
// staged in LDS as 16-bit fixed point by transposing reads
// (ds_read_b64_tr_b16): in each 16-lane group lane j reads the 4-dim codebook
// row of (token j/4, value block 8*(j%4) + nt), and the read hands lane i the
// column i of that 4 x 16 block, i.e. dim i%4 of block 8*(i/4) + nt for the 4
// tokens -- the B operand's codes.  Each codebook dim (value block, dim j)
// holds u = rint((C - zero)/scale) with zero = min, scale = (max - min)/65535
// over its centroids, so |C - (zero + scale*u)| <= scale/2 (an fp16 copy of C
// leaves up to 2^-11 |C|, which at 131072 tokens of N(0,1) values came to
// 1.1e-3 of the output).  The code's bytes u = 256 h + l enter as two fp16
// operands of the same product, each byte placed under a constant exponent
// byte by one v_perm_b32: 0x78hh = 32768 + 32 h and 0x58ll = 128 + l/8, both
// exact, so the accumulator sums p (32896 + u/8); one rounding per product
// of 32 tokens keeps that offset's cost to a few 1e-5 of the output (fp32
// emulation at 131072 tokens: 1.6e-4 of the output in all, 1.3e-4 of it the
// codes' own step).  The combine turns the sums into p-weighted values with
// each dim's scale and zero.  MFMA
// column n of n-tile nt therefore holds codec dim ((8*(n/4) + nt)*4 + n%4),
// and a lane's eight n-tiles read index bytes 8*(n%4) .. +7 of one token, an
// 8-byte load per 16 tokens.  The heavy-dim dot products run on
// v_mfma_f32_4x4x4f16 (16 blocks of 4 tokens: A = the 4 query rows' heavy
// dims, B = each token's own fp16 heavy dims, D = the token's 4 row scores in
// its own lane), with an fp16 hi/lo split of the query unless it is already
// fp16.  There is no loader wave and no LDS ring: each wave loads its next
// 64-token unit (index rows, heavy keys, value indices) into registers while
// it computes the current one (that load is clamped to the split's last unit
// rather than skipped, so the loop stays straight-line and the wait for a
// unit's data is a plain vmcnt).  The workgroup writes its split's
// (m, l, acc) partials, or with one split the fp32 rows, in the codec basis,
// for the transformed-basis merge.
// ---------------------------------------------------------------------------
constexpr int kSvNB = 16;    // key blocks of head_dim 128
constexpr int kSvNBV = 32;   // value blocks of block_dim 4
constexpr int kSvD = 128;
constexpr int kSvWaves = 8;
constexpr int kSvVcbBytes = kSvNBV * 256 * 8;  // u16 codes [value block][256][4], at LDS offset 0
constexpr int kSvLutBytes = kSvNB * 256 * 16;  // float4 (4 rows) [key block][256]
constexpr int kSvPstBytes = kSvWaves * 8 * kPStride * 2;
constexpr int kSvSzBytes = kSvD * 2 * 4;      // per codebook dim: zero, scale (f32)
constexpr int kSvLdsBytes = kSvVcbBytes + kSvLutBytes + kSvPstBytes + kSvSzBytes;
// the code bytes' fp16 operand patterns: 0x78hh = 32768 + 32 h, 0x58ll = 128 + l / 8
constexpr uint32_t kSvHiPat = 0x78787878u, kSvLoPat = 0x58585858u;
constexpr float kSvCodeOff = -32896.f;  // the operands sum to u/8 - kSvCodeOff
static_assert(kSvLdsBytes <= kLdsMax, "SunShape-value MFMA LDS budget");
static_assert(kSvVcbBytes <= 65536, "value codebook addressed with 16-bit LDS offsets");

// ds_read_b64_tr_b16 at LDS byte offset `off` of the dynamic LDS block: in
// each 16-lane group, lane j reads 4 halves; lane i receives column i of the
// 4 x 16 block they form (row r from lane 4r + i/4, element i%4).
__device__ __forceinline__ f16x4 ds_read_tr16(const char *lds_base, uint32_t off) {
    typedef __attribute__((__vector_size__(4 * sizeof(__fp16)))) __fp16 hf16x4;
    typedef __attribute__((address_space(3))) hf16x4 lhf16x4;
    lhf16x4 *p = (lhf16x4 *)(static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds_base)) + off);
    return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(p));
}

template <int NH8>
struct SvUnit {
    uint4 k;                          // key index row of token t0 + lane
    uint4 kh[NH8 > 0 ? NH8 : 1];      // its heavy key dims (fp16)
    uint2 vi[4];                      // value index bytes 8*(l16%4) .. +7 of token 16ks + 4g + l16/4
};

template <int NH8>
__global__ void __launch_bounds__(kSvWaves * kWave)
    sunv_mfma_kernel(DecodeCommon c, typename VSunV<128, 4>::Args va) {
    constexpr int NC = kSvWaves, TH = NC * kWave, R = kMfmaRows, D = kSvD;
    extern __shared__ __align__(16) float4 smem4[];
    char *smem = reinterpret_cast<char *>(smem4);
    uint2 *vcb = reinterpret_cast<uint2 *>(smem);                            // [32][256]
    float4 *lut4 = reinterpret_cast<float4 *>(smem + kSvVcbBytes);           // [16][256]
    _Float16 *pst = reinterpret_cast<_Float16 *>(smem + kSvVcbBytes + kSvLutBytes);
    float *vsz = reinterpret_cast<float *>(smem + kSvVcbBytes + kSvLutBytes + kSvPstBytes);  // [D][2]
    const lds_t<f32x4> *lut_l = (const lds_t<f32x4> *)(smem + kSvVcbBytes);

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int col = blockIdx.y;
    const int split = blockIdx.x;
    const int rg = col % c.n_rg;
    const int kvh = (col / c.n_rg) % c.n_kv_heads;
    const int64_t bb = col / (c.n_rg * c.n_kv_heads);
    const int64_t bh = bb * c.n_kv_heads + kvh;
    auto row_off = [&](int r) -> int64_t {
        const int64_t gr = (int64_t)rg * R + r;
        const int64_t rr = gr / c.t_q, tq = gr - rr * c.t_q;
        return ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
    };
    auto row_ok = [&](int r) -> bool { return (int64_t)rg * R + r < c.rows_total; };

    // 1. query rows round_to(q_dtype, q * scale), permuted (attention.py:208,
    //    228), staged in the P area; heavy blocks of the codec
    float *qp = reinterpret_cast<float *>(pst);  // [R][D], 2 KB of the P area
    for (int i = tid; i < R * D; i += TH) {
        const int r = i / D, j = i - r * D;
        float x = 0.f;
        if (row_ok(r)) {
            const int src = c.perm ? min(max(c.perm[j], 0), D - 1) : j;
            x = round_to(c.q_dtype, load_as_f32(c.q, c.q_dtype, row_off(r) + src) * c.scale);
        }
        qp[i] = x;
    }
    uint32_t heavy_blocks = 0;
    for (int j = 0; j < NH8 * 8; ++j)
        heavy_blocks |= 1u << (min(max(va.heavy_dims[j], 0), D - 1) / kBlockDim);
    // value codebook -> 16-bit codes.  Each codebook dim d = 4 vb + j takes
    // zero = min, scale = (max - min) / 65535 over its n_centroids entries:
    // four adjacent threads scan a quarter of them each and combine
    {
        static_assert(TH == 4 * D, "four threads per codebook dim");
        const int d = tid >> 2, part = tid & 3, vb = d >> 2, j = d & 3;
        const float *col_p = va.cb + (int64_t)vb * va.n_centroids * 4 + j;
        float lo = INFINITY, hi = -INFINITY;
        for (int cc = part; cc < va.n_centroids; cc += 4) {
            const float x = col_p[(int64_t)cc * 4];
            lo = fminf(lo, x);
            hi = fmaxf(hi, x);
        }
        lo = fminf(lo, __shfl_xor(lo, 1));
        hi = fmaxf(hi, __shfl_xor(hi, 1));
        lo = fminf(lo, __shfl_xor(lo, 2));
        hi = fmaxf(hi, __shfl_xor(hi, 2));
        if (part == 0) {
            const bool ok = va.n_centroids > 0 && hi > lo;
            vsz[2 * d] = va.n_centroids > 0 ? lo : 0.f;
            vsz[2 * d + 1] = ok ? (hi - lo) * (1.f / 65535.f) : 0.f;
        }
    }
    __syncthreads();
    for (int i = tid; i < kSvNBV * 256; i += TH) {
        const int vb = i >> 8, cc = i & 255;
        uint32_t uc[4] = {0u, 0u, 0u, 0u};
        if (cc < va.n_centroids) {
            const float4 v =
                *reinterpret_cast<const float4 *>(va.cb + ((int64_t)vb * va.n_centroids + cc) * 4);
            const float x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float z = vsz[2 * (4 * vb + j)], sc = vsz[2 * (4 * vb + j) + 1];
                const float q = sc > 0.f ? rintf(__fdiv_rn(x[j] - z, sc)) : 0.f;
                uc[j] = (uint32_t)fminf(fmaxf(q, 0.f), 65535.f);
            }
        }
        vcb[i] = make_uint2(uc[0] | (uc[1] << 16), uc[2] | (uc[3] << 16));
    }
    __syncthreads();
    // 2. LUT[b][cc] = the 4 rows' q'[b-block] . C[b][cc] in log2 units
    //    (kernels.py:178-190); heavy blocks score from their fp16 keys: 0
    for (int e = tid; e < kSvNB * c.n_centroids; e += TH) {
        const int b = e / c.n_centroids, cc = e - b * c.n_centroids;
        const float4 *cp = reinterpret_cast<const float4 *>(c.centroids + (int64_t)e * kBlockDim);
        const float4 c0 = cp[0], c1 = cp[1];
        float dt[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float *qr = qp + r * D + b * kBlockDim;
            float dot = qr[0] * c0.x;
            dot = fmaf(qr[1], c0.y, dot);
            dot = fmaf(qr[2], c0.z, dot);
            dot = fmaf(qr[3], c0.w, dot);
            dot = fmaf(qr[4], c1.x, dot);
            dot = fmaf(qr[5], c1.y, dot);
            dot = fmaf(qr[6], c1.z, dot);
            dot = fmaf(qr[7], c1.w, dot);
            dt[r] = ((heavy_blocks >> b) & 1u) ? 0.f : dot * kLog2e;
        }
        lut4[b * 256 + cc] = make_float4(dt[0], dt[1], dt[2], dt[3]);
    }
    // A operands of the heavy-dim products: query row lane%4, heavy dims
    // 4kk .. 4kk+3, as fp16 hi and (scaled by 2^11) lo parts; non-fp16 rows
    // scaled by 2^-s_r so the hi parts stay in range (products times 2^s_r)
    const bool qsplit = c.q_dtype != SS_F16;
    f32x4 qsc = f32x4{1.f, 1.f, 1.f, 1.f};
    float qinv = 1.f;
    if (NH8 > 0 && qsplit) {
        float mx = 0.f;
        for (int j = l16; j < D; j += 16) mx = fmaxf(mx, fabsf(qp[g * D + j]));
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        const int sh = row_exp_shift(mx);
        qsc = f32x4{exp2i(__shfl(sh, 0)), exp2i(__shfl(sh, 16)), exp2i(__shfl(sh, 32)),
                    exp2i(__shfl(sh, 48))};
        qinv = exp2i(-__shfl(sh, 16 * (lane & 3)));
    }
    f16x4 ah[NH8 > 0 ? 2 * NH8 : 1], al[NH8 > 0 ? 2 * NH8 : 1];
    if constexpr (NH8 > 0) {
#pragma unroll
        for (int kk = 0; kk < 2 * NH8; ++kk)
#pragma unroll
            for (int e2 = 0; e2 < 4; ++e2) {
                const int hd = min(max(va.heavy_dims[4 * kk + e2], 0), D - 1);
                const float x = qp[(lane & 3) * D + hd] * qinv;
                const _Float16 h = (_Float16)x;
                ah[kk][e2] = h;
                al[kk][e2] = (_Float16)((x - (float)h) * kSplitScale);
            }
    }
    __syncthreads();  // LUT and codebook staged, query read; the P area is free

    // 3. this split's 64-token units, wave wv taking units wv, wv + NC, ...
    const int64_t t_beg = (int64_t)split * c.tiles_per_split * kWave;
    const int64_t t_end = min(c.t_kv, t_beg + (int64_t)c.tiles_per_split * kWave);
    const int n_units = t_end > t_beg ? (int)((t_end - t_beg + kWave - 1) / kWave) : 0;
    const int64_t t_last = max(t_end - 1, (int64_t)0);
    const uint8_t *idx_head = c.idx + bh * c.cap * kSvNB;
    const int64_t vrow0 = bh * c.cap;
    const int q4 = l16 >> 2, w4 = l16 & 3;
    // bytes: codebook row (block 8*w4 + nt, byte) this lane reads for the
    // transposing gather (nt * 2048 goes in the instruction's offset)
    const uint32_t vbase = (uint32_t)(8 * w4) * 256 * 8;

    int64_t lim[R];
    int64_t lim_min = INT64_MAX;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t gr = (int64_t)rg * R + r;
        lim[r] = !row_ok(r) ? -1 : c.causal ? c.q_offset + (gr % c.t_q) : INT64_MAX;
        lim_min = min(lim_min, lim[r]);
    }

    // token offsets within the head are 32-bit (cap < 2^26 checked on the
    // host), so each load is a uniform base plus one 32-bit lane offset
    const char *kidx_b = reinterpret_cast<const char *>(idx_head);
    const char *kh_b = reinterpret_cast<const char *>(va.kheavy + (NH8 > 0 ? vrow0 * (NH8 * 8) : 0));
    const char *vi_b = reinterpret_cast<const char *>(va.idx + vrow0 * kSvNBV);
    const uint32_t t_last32 = (uint32_t)t_last;
    auto at = [](const char *base, uint32_t byte_off) { return base + byte_off; };
    auto load_unit = [&](SvUnit<NH8> &U, int u) {
        const uint32_t t0 = (uint32_t)t_beg + (uint32_t)u * kWave;
        const uint32_t tk = min(t0 + (uint32_t)lane, t_last32);
        U.k = *reinterpret_cast<const uint4 *>(at(kidx_b, tk * kSvNB));
        if constexpr (NH8 > 0) {
#pragma unroll
            for (int j = 0; j < NH8; ++j)
                U.kh[j] = *reinterpret_cast<const uint4 *>(at(kh_b, tk * (NH8 * 16) + j * 16));
        }
        const uint32_t tg = t0 + 4u * g + (uint32_t)q4;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
            U.vi[ks] = *reinterpret_cast<const uint2 *>(
                at(vi_b, min(tg + 16u * ks, t_last32) * kSvNBV + 8u * w4));
    };

    float m[R], lsum[R];
    f32x4 acc[8];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        m[r] = -1e30f;
        lsum[r] = 0.f;
    }
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    _Float16 *pw = pst + wv * 8 * kPStride;

    auto compute_unit = [&](const SvUnit<NH8> &cur, int u) {
        const int64_t t0 = t_beg + (int64_t)u * kWave;
        const int n_in = (int)min(t_end - t0, (int64_t)kWave);
        // scores: the 16 LUT reads in flight at once, then a tree sum
        f32x4 e[kSvNB];
#pragma unroll
        for (int b = 0; b < kSvNB; ++b) {
            const uint32_t w = b < 4 ? cur.k.x : b < 8 ? cur.k.y : b < 12 ? cur.k.z : cur.k.w;
            e[b] = lut_l[b * 256 + __builtin_amdgcn_ubfe(w, (b & 3) * 8, 8)];
        }
#pragma unroll
        for (int w = 1; w < kSvNB; w *= 2)
#pragma unroll
            for (int b = 0; b < kSvNB; b += 2 * w) e[b] += e[b + w];
        f32x4 s4 = e[0];
        if constexpr (NH8 > 0) {
            // heavy dims on the matrix cores: D[row][token lane] in this lane
            f32x4 hs = f32x4{0.f, 0.f, 0.f, 0.f}, hl = hs;
#pragma unroll
            for (int j = 0; j < NH8; ++j) {
                const uint4 kv = cur.kh[j];
                const f16x4 b0 = __builtin_bit_cast(f16x4, make_uint2(kv.x, kv.y));
                const f16x4 b1 = __builtin_bit_cast(f16x4, make_uint2(kv.z, kv.w));
                hs = __builtin_amdgcn_mfma_f32_4x4x4f16(ah[2 * j], b0, hs, 0, 0, 0);
                hs = __builtin_amdgcn_mfma_f32_4x4x4f16(ah[2 * j + 1], b1, hs, 0, 0, 0);
            }
            if (qsplit) {
#pragma unroll
                for (int j = 0; j < NH8; ++j) {
                    const uint4 kv = cur.kh[j];
                    const f16x4 b0 = __builtin_bit_cast(f16x4, make_uint2(kv.x, kv.y));
                    const f16x4 b1 = __builtin_bit_cast(f16x4, make_uint2(kv.z, kv.w));
                    hl = __builtin_amdgcn_mfma_f32_4x4x4f16(al[2 * j], b0, hl, 0, 0, 0);
                    hl = __builtin_amdgcn_mfma_f32_4x4x4f16(al[2 * j + 1], b1, hl, 0, 0, 0);
                }
            }
            s4 += (hs + hl * (1.f / kSplitScale)) * (qsc * kLog2e);
        }
        float sc[R] = {s4.x, s4.y, s4.z, s4.w};
        bool moved = true;
        if (n_in == kWave && t0 + (kWave - 1) <= lim_min) {
            uint64_t above = 0;
#pragma unroll
            for (int r = 0; r < R; ++r) above |= __builtin_amdgcn_ballot_w64(sc[r] > m[r] + kPLag);
            moved = above != 0;
        } else {
            const bool kok = lane < n_in;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int lim_rel = (int)max(min(lim[r] - t0, (int64_t)kWave), (int64_t)-1);
                sc[r] += (kok && lane <= lim_rel) ? 0.f : -INFINITY;
            }
        }
        float corr[R], p[R];
        if (moved) {
            float tmax[R];
            wave_max4_dpp(sc, tmax);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float mn = fmaxf(m[r], tmax[r]);
                corr[r] = fast_exp2(m[r] - mn);
                p[r] = fast_exp2(sc[r] - mn);
                lsum[r] = fmaf(lsum[r], corr[r], p[r]);
                m[r] = mn;
            }
        } else {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                corr[r] = 1.f;
                p[r] = fast_exp2(sc[r] - m[r]);
                lsum[r] += p[r];
            }
        }
        // P as fp16 hi/lo rows (A rows 0-3 hi, 4-7 lo, 8-15 zero)
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const float x = p[r] * kPScale;
            const _Float16 hi = (_Float16)x;
            pw[r * kPStride + lane] = hi;
            pw[(r + 4) * kPStride + lane] = (_Float16)(x - (float)hi);
        }
        wave_lds_sync();
        if (moved) {
            const f32x4 cv4 = f32x4{corr[0], corr[1], corr[2], corr[3]};
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) acc[nt] *= cv4;
        }
        const bool a_live = l16 < 8;
        // v_mfma_f32_16x16x32_f16 (full fp16 rate) over two 16-token k-steps:
        // K slots 8g .. 8g+3 of lane l are tokens 16(2k2) + 4g + 0..3, slots
        // 8g+4 .. 8g+7 tokens 16(2k2+1) + 4g + 0..3, in A (its P row) and in
        // B (the two transposing reads)
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            f16x4 a0 = f16x4{0, 0, 0, 0}, a1 = a0;
            if (a_live) {
                a0 = *reinterpret_cast<const f16x4 *>(pw + l16 * kPStride + 32 * k2 + 4 * g);
                a1 = *reinterpret_cast<const f16x4 *>(pw + l16 * kPStride + 32 * k2 + 16 + 4 * g);
            }
            const f16x8 a = __builtin_shufflevector(a0, a1, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const uint2 w0 = cur.vi[2 * k2], w1 = cur.vi[2 * k2 + 1];
                const uint32_t b0 = __builtin_amdgcn_ubfe(nt < 4 ? w0.x : w0.y, (nt & 3) * 8, 8);
                const uint32_t b1 = __builtin_amdgcn_ubfe(nt < 4 ? w1.x : w1.y, (nt & 3) * 8, 8);
                const uint2 c0 = __builtin_bit_cast(uint2, ds_read_tr16(smem, vbase + b0 * 8 + nt * 2048));
                const uint2 c1 = __builtin_bit_cast(uint2, ds_read_tr16(smem, vbase + b1 * 8 + nt * 2048));
                // codes u (two per word) -> operands 32768 + 32 h and 128 + l / 8:
                // v_perm_b32 places each code byte under its exponent byte
                // (selector bytes 0-3 pick the code word's bytes, 4 the pattern's)
                const uint32_t cw[4] = {c0.x, c0.y, c1.x, c1.y};
                uint32_t bh[4], bl[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bh[q] = __builtin_amdgcn_perm(kSvHiPat, cw[q], 0x04030401u);
                    bl[q] = __builtin_amdgcn_perm(kSvLoPat, cw[q], 0x04020400u);
                }
                const f16x8 bop_h = __builtin_bit_cast(f16x8, make_uint4(bh[0], bh[1], bh[2], bh[3]));
                const f16x8 bop_l = __builtin_bit_cast(f16x8, make_uint4(bl[0], bl[1], bl[2], bl[3]));
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop_h, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop_l, acc[nt], 0, 0, 0);
            }
        }
        wave_lds_sync();
    };
    // two register sets in turn: the next unit's loads are issued before the
    // current unit is computed
    SvUnit<NH8> ua, ub;
    if (wv < n_units) load_unit(ua, wv);
    for (int u = wv; u < n_units; u += 2 * NC) {
        load_unit(ub, min(u + NC, n_units - 1));
        compute_unit(ua, u);
        if (u + NC >= n_units) break;
        load_unit(ua, min(u + 2 * NC, n_units - 1));
        compute_unit(ub, u + NC);
    }

    // 4. the workgroup combine: waves' (m, l) and (hi, lo) accumulators in
    //    LDS (over the LUT, which no wave reads any more)
    {
        float ls[R];
        wave_sum4_dpp(lsum, ls);
#pragma unroll
        for (int r = 0; r < R; ++r) lsum[r] = ls[r];
    }
    __syncthreads();
    float *wm = reinterpret_cast<float *>(smem + kSvVcbBytes);  // [NC][R]
    float *wl = wm + NC * R;                                     // [NC][R]
    float *wa = wl + NC * R;                                     // [NC][2][R][D]
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            wm[wv * R + r] = m[r];
            wl[wv * R + r] = lsum[r];
        }
    }
    if (g < 2) {
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
            const int d = (8 * q4 + nt) * 4 + w4;
#pragma unroll
            for (int r = 0; r < R; ++r)
                wa[((wv * 2 + g) * R + r) * D + d] = acc[nt][r] * (1.f / kPScale);
        }
    }
    __syncthreads();
    const int S = c.n_splits;
    for (int i = tid; i < R * D; i += TH) {
        const int r = i / D, d = i - r * D;
        float M = -1e30f;
#pragma unroll
        for (int w = 0; w < NC; ++w) M = fmaxf(M, wm[w * R + r]);
        float L = 0.f, A = 0.f;
#pragma unroll
        for (int w = 0; w < NC; ++w) {
            const float f = fast_exp2(wm[w * R + r] - M);
            L = fmaf(wl[w * R + r], f, L);
            A = fmaf(wa[((w * 2) * R + r) * D + d] + wa[((w * 2 + 1) * R + r) * D + d], f, A);
        }
        // sum p (u/8 - kSvCodeOff) -> sum p C = (zero + 8 kSvCodeOff scale) L + 8 scale A
        {
            const float z = vsz[2 * d], sc = vsz[2 * d + 1];
            A = fmaf(8.f * sc, A, (z + (8.f * kSvCodeOff) * sc) * L);
        }
        if (S == 1) {
            if (row_ok(r)) store_from_f32(c.out, c.out_dtype, row_off(r) + d, L > 0.f ? A / L : 0.f);
        } else {
            const int64_t slot = ((int64_t)col * S + split) * R + r;
            c.part_acc[slot * D + d] = A;
            if (d == 0) *reinterpret_cast<float2 *>(c.part_ml + slot * 2) = make_float2(M, L);
        }
    }
}

// ---------------------------------------------------------------------------
// Merge of split-T partials: one workgroup per (group, row).  One wave turns
// the splits' (m, l) into weights exp2(m_s - M) and the merged l; every thread
// then streams float4 slices of the accumulators of a subset of splits (loads
// issued back to back) and the slices are reduced in LDS.  Runs as its own
// launch: a cross-workgroup hand-off inside one kernel needs an agent-scope L2
// write-back per workgroup on multi-XCD CDNA parts.
template <int D>
__global__ void __launch_bounds__(kDecodeThreads)
    decode_merge_kernel(DecodeCommon c, int R, const float *rot, void *rot_out, int rot_dtype) {
    constexpr int CH = D / 4;                // float4 chunks of one output row
    constexpr int NP = kDecodeThreads / CH;  // split partitions
    __shared__ float wsh[kMaxSplits];
    __shared__ float lsh;
    __shared__ float4 red[NP * CH];
    __shared__ float yrow[D];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid >> 6;
    const int col = blockIdx.x, r = blockIdx.y;
    const int64_t gr = (int64_t)(col % c.n_rg) * R + r;
    if (gr >= c.rows_total) return;  // uniform over the workgroup
    const int S = c.n_splits;
    const int kvh = (col / c.n_rg) % c.n_kv_heads;
    const int64_t bb = col / (c.n_rg * c.n_kv_heads);
    const float *ml = c.part_ml + ((int64_t)col * S * R + r) * 2;
    if (wv == 0) {
        float M = -1e30f;
        for (int s2 = lane; s2 < S; s2 += kWave) M = fmaxf(M, ml[(int64_t)s2 * R * 2]);
        M = wave_max(M);
        float L = 0.f;
        for (int s2 = lane; s2 < S; s2 += kWave) {
            const float2 v = *reinterpret_cast<const float2 *>(ml + (int64_t)s2 * R * 2);
            const float w = fast_exp2(v.x - M);
            wsh[s2] = w;
            L = fmaf(v.y, w, L);
        }
        L = wave_sum(L);
        if (lane == 0) lsh = L;
    }
    __syncthreads();
    {
        const int chunk = tid % CH, part = tid / CH;
        const float4 *ap =
            reinterpret_cast<const float4 *>(c.part_acc + ((int64_t)col * S * R + r) * D) + chunk;
        float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
        for (int s2 = part; s2 < S; s2 += NP) {
            const float4 v = ap[(int64_t)s2 * R * CH];
            const float w = wsh[s2];
            a.x = fmaf(v.x, w, a.x);
            a.y = fmaf(v.y, w, a.y);
            a.z = fmaf(v.z, w, a.z);
            a.w = fmaf(v.w, w, a.w);
        }
        red[part * CH + chunk] = a;
    }
    __syncthreads();
    if (tid < D) {
        const int d = tid, chunk = d >> 2;
        float A = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float4 v = red[p * CH + chunk];
            A += (d & 3) == 0 ? v.x : (d & 3) == 1 ? v.y : (d & 3) == 2 ? v.z : v.w;
        }
        const int64_t rr = gr / c.t_q, tq = gr - rr * c.t_q;
        const int64_t off = ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
        const float y = lsh > 0.f ? A / lsh : 0.f;
        if (rot)
            yrow[d] = y;
        else
            store_from_f32(c.out, c.out_dtype, off + d, y);
    }
    if (rot) {
        // the merged row is in a transformed basis (TurboQuant rotation, a
        // value codec's permutation or rotation): out = y @ M.  Every thread
        // takes one output dim and a contiguous share of k (two interleaved
        // accumulators), reading row k of M coalesced over the dims; the
        // shares are added in LDS.
        constexpr int PARTS = kDecodeThreads / D, KP = D / PARTS;
        __shared__ float rsum[PARTS][D];
        __syncthreads();
        {
            const int dd = tid % D, part = tid / D, k0 = part * KP;
            float a0 = 0.f, a1 = 0.f;
#pragma unroll 8
            for (int k = k0; k < k0 + KP; k += 2) {
                a0 = fmaf(yrow[k], rot[k * D + dd], a0);
                a1 = fmaf(yrow[k + 1], rot[(k + 1) * D + dd], a1);
            }
            rsum[part][dd] = a0 + a1;
        }
        __syncthreads();
        if (tid < D) {
            const int64_t rr = gr / c.t_q, tq = gr - rr * c.t_q;
            const int64_t off = ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
            float a = 0.f;
#pragma unroll
            for (int pp = 0; pp < PARTS; ++pp) a += rsum[pp][tid];
            store_from_f32(rot_out, rot_dtype, off + tid, a);
        }
    }
}

// out[row] = y[row] @ rot for fp32 rows of the rotated basis (the TurboQuant
// dequant's `unit = C[idx] @ R`, value_codecs.py:173-177, applied once to the
// attention output).  A workgroup takes kRotRows rows: thread (part, d) sums
// rows part*RPT .. +RPT-1 of column d over k in order, reading R row k
// (coalesced over d) once per k.
constexpr int kRotRows = 16;
template <int D>
__global__ void __launch_bounds__(256)
    rotate_rows_kernel(const float *y, const float *rot, int64_t rows, void *out, int out_dtype) {
    constexpr int PARTS = 256 / D;
    constexpr int RPT = kRotRows / PARTS;
    __shared__ float ys[kRotRows][D];
    const int64_t r0 = (int64_t)blockIdx.x * kRotRows;
    for (int i = threadIdx.x; i < kRotRows * D; i += 256) {
        const int64_t r = r0 + i / D;
        ys[i / D][i % D] = r < rows ? y[r * D + i % D] : 0.f;
    }
    __syncthreads();
    const int d = threadIdx.x % D, part = threadIdx.x / D;
    float acc[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) acc[j] = 0.f;
    for (int k = 0; k < D; ++k) {
        const float rk = rot[k * D + d];
#pragma unroll
        for (int j = 0; j < RPT; ++j) acc[j] = fmaf(ys[part * RPT + j][k], rk, acc[j]);
    }
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int64_t r = r0 + part * RPT + j;
        if (r < rows) store_from_f32(out, out_dtype, r * D + d, acc[j]);
    }
}

// A hybrid cache's buffered tokens (original basis, element j of token t of
// (b, h) at buf[b*sb + h*sh + t*st + j]) as split partial `slot` of the
// TurboQuant decode, so they join the compressed tokens' softmax in the merge
// (the reference runs its two-pass path instead, attention.py:307-350).  One
// workgroup per column.  Scores are fp32 dot products with the unpermuted
// scaled query, in log2 units, at positions t_kv + t; online softmax over
// chunks of 256 tokens; P.V in the original basis.  The accumulators are then
// taken into the rotated basis, acc @ R^T (R orthogonal), where the merge
// adds them to the compressed splits' before the output rotation; with no
// R (rot null: values in the original basis) they are stored as they are.
template <int D, int R>
__global__ void __launch_bounds__(256)
    buffer_partial_kernel(DecodeCommon c, const void *kbuf, const void *vbuf, int buf_dtype,
                          int64_t sb, int64_t sh, int64_t st, int64_t t_buf, const float *rot,
                          int slot) {
    constexpr int T = 256, NW = T / kWave;
    __shared__ float qs[R][D];
    __shared__ float pr[R][T];
    __shared__ float red[NW][R];
    __shared__ float acc_s[R][D];
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wv = tid >> 6;
    const int col = blockIdx.x;
    const int rg = col % c.n_rg;
    const int kvh = (col / c.n_rg) % c.n_kv_heads;
    const int64_t bb = col / (c.n_rg * c.n_kv_heads);
    auto row_ok = [&](int r) { return (int64_t)rg * R + r < c.rows_total; };
    auto row_off = [&](int r) -> int64_t {
        const int64_t g = (int64_t)rg * R + r;
        const int64_t rr = g / c.t_q, tq = g - rr * c.t_q;
        return ((bb * c.n_q_heads + kvh * c.rep + rr) * c.t_q + tq) * D;
    };
    for (int i = tid; i < R * D; i += T) {
        const int r = i / D, j = i - r * D;
        qs[r][j] = row_ok(r) ? round_to(c.q_dtype, load_as_f32(c.q, c.q_dtype, row_off(r) + j) *
                                                        c.scale)
                             : 0.f;
    }
    int64_t lim[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t g = (int64_t)rg * R + r;
        lim[r] = !row_ok(r) ? -1 : c.causal ? c.q_offset + (g % c.t_q) : INT64_MAX;
    }
    const int64_t base = bb * sb + kvh * sh;
    // thread (r, d) of the P.V: rows r = tid / D + k * (T / D)
    constexpr int RPT = (R * D + T - 1) / T;
    float m[R], l[R], acc[RPT];
#pragma unroll
    for (int r = 0; r < R; ++r) m[r] = -1e30f, l[r] = 0.f;
#pragma unroll
    for (int k = 0; k < RPT; ++k) acc[k] = 0.f;
    __syncthreads();
    for (int64_t j0 = 0; j0 < t_buf; j0 += T) {
        const int64_t j = j0 + tid;
        float s[R];
#pragma unroll
        for (int r = 0; r < R; ++r) s[r] = 0.f;
        if (j < t_buf) {
            for (int d = 0; d < D; ++d) {
                const float kv = load_as_f32(kbuf, buf_dtype, base + j * st + d);
#pragma unroll
                for (int r = 0; r < R; ++r) s[r] = fmaf(qs[r][d], kv, s[r]);
            }
        }
        float cm[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const bool ok = j < t_buf && c.t_kv + j <= lim[r];
            s[r] = ok ? s[r] * kLog2e : -INFINITY;
            cm[r] = wave_max(s[r]);
        }
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) red[wv][r] = cm[r];
        __syncthreads();
        float corr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float mx = red[0][r];
#pragma unroll
            for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red[w][r]);
            const float mn = fmaxf(m[r], mx);
            corr[r] = fast_exp2(m[r] - mn);
            m[r] = mn;
            pr[r][tid] = fast_exp2(s[r] - mn);
        }
        __syncthreads();  // probabilities staged; red free
        float ps[R];
#pragma unroll
        for (int r = 0; r < R; ++r) ps[r] = wave_sum(pr[r][tid]);
        if (lane == 0)
#pragma unroll
            for (int r = 0; r < R; ++r) red[wv][r] = ps[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float sum = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) sum += red[w][r];
            l[r] = fmaf(l[r], corr[r], sum);
        }
        const int n = (int)min((int64_t)T, t_buf - j0);
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
            const int e = tid + k * T;
            if (e < R * D) {
                const int r = e / D, d = e - r * D;
                float a = acc[k] * corr[r];
                for (int i = 0; i < n; ++i)
                    a = fmaf(pr[r][i], load_as_f32(vbuf, buf_dtype, base + (j0 + i) * st + d), a);
                acc[k] = a;
            }
        }
        __syncthreads();  // pr and red reused by the next chunk
    }
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int e = tid + k * T;
        if (e < R * D) acc_s[e / D][e % D] = acc[k];
    }
    __syncthreads();
    const int64_t slot0 = ((int64_t)col * c.n_splits + slot) * R;
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
        const int e = tid + k * T;
        if (e < R * D) {
            const int r = e / D, kk = e - r * D;
            float a = 0.f;
            if (rot)
                for (int d = 0; d < D; ++d) a = fmaf(acc_s[r][d], rot[kk * D + d], a);
            else
                a = acc_s[r][kk];
            c.part_acc[(slot0 + r) * D + kk] = a;
            if (kk == 0)
                *reinterpret_cast<float2 *>(c.part_ml + (slot0 + r) * 2) = make_float2(m[r], l[r]);
        }
    }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct DecodeShape {
    int R, n_rg, n_cols, S, tiles_per_split;
};

static int rows_per_group(int64_t rows_total) { return rows_total <= 1 ? 1 : 4; }

// Kernel families: the VALU kernel (any value layout/dtype, 4 waves per
// workgroup, 1 or 4 rows) and the MFMA kernel (fp16 values 8-token
// interleaved, 4 or 8 compute waves plus a loader wave, 4 rows).
// kKindSunv: the matrix-core SunShape-value decode (one 136 KB-LDS
// workgroup per compute unit, eight waves)
enum DecodeKind { kKindValu = 0, kKindMfma = 1, kKindSunv = 2 };
constexpr int kMfmaWaves = 4;  // fewest compute waves of an MFMA kernel (tiles per split)

static DecodeShape decode_shape(int64_t batch, int hq, int hkv, int64_t t_q, int64_t t_kv,
                                int n_splits, int kind = kKindValu) {
    DecodeShape s;
    const int64_t rows = (int64_t)(hq / hkv) * t_q;
    s.R = kind == kKindMfma ? kMfmaRows : rows_per_group(rows);
    s.n_rg = (int)((rows + s.R - 1) / s.R);
    s.n_cols = (int)(batch * hkv * s.n_rg);
    const int64_t tiles = (t_kv + kWave - 1) / kWave;
    const int waves = kind == kKindMfma ? kMfmaWaves : kind == kKindSunv ? 8 : kDecodeWaves;
    int S = n_splits;
    if (S <= 0) {
        // about one (MFMA) or two (VALU) workgroups per compute unit, each
        // with at least one 64-token tile per wave
        const int64_t target = (kind == kKindValu ? 2LL : 1LL) * device_cu_count();
        int64_t want = (target + s.n_cols - 1) / s.n_cols;
        const int64_t cap = tiles / waves;
        if (want > cap) want = cap;
        S = (int)(want < 1 ? 1 : want);
    }
    if (tiles == 0) S = 1;
    if (S > tiles && tiles > 0) S = (int)tiles;
    if (S > kMaxSplits) S = kMaxSplits;
    s.tiles_per_split = tiles > 0 ? (int)((tiles + S - 1) / S) : 0;
    if (s.tiles_per_split > 0) S = (int)((tiles + s.tiles_per_split - 1) / s.tiles_per_split);
    s.S = S;
    return s;
}

// Workspace layout: [part_cnt: kCntBytes, one int per column, spread out]
//                   [part_ml: n_cols*S*R float2, padded to 256 B]
//                   [part_acc: n_cols*S*R*D float]
// The MFMA path counts finished splits per column in part_cnt and its last
// split resets the count.  The counter area has the same place and size for
// every shape, so it must be zero before the first call on a workspace and
// then stays zero between calls; shapes with more than kCntBytes/4 columns
// merge with a separate launch instead.
constexpr size_t kCntBytes = 64 * 1024;
struct WsLayout {
    size_t cnt, ml, acc, total;
};

static WsLayout ws_layout(const DecodeShape &s, int head_dim) {
    auto pad = [](size_t b) { return (b + 255) / 256 * 256; };
    WsLayout w;
    const size_t slots = (size_t)s.n_cols * s.S * s.R;
    w.cnt = 0;
    w.ml = kCntBytes;
    w.acc = w.ml + pad(slots * 2 * sizeof(float));
    w.total = w.acc + slots * head_dim * sizeof(float);
    return w;
}

static size_t decode_ws_bytes(const DecodeShape &s, int head_dim) {
    return s.S <= 1 ? 0 : ws_layout(s, head_dim).total;
}

template <int D>
static int launch_merge(const DecodeCommon &c, const DecodeShape &s, hipStream_t st,
                        const float *rot = nullptr, void *rot_out = nullptr, int rot_dtype = 0) {
    if (s.S <= 1) return SS_OK;
    auto merge = decode_merge_kernel<D>;
    hipLaunchKernelGGL(merge, dim3(s.n_cols, s.R), dim3(kDecodeThreads), 0, st, c, s.R, rot,
                       rot_out, rot_dtype);
    SS_LAUNCH_CHECK("decode_merge_kernel launch");
    return SS_OK;
}

// Once per instance of the matrix-core decode kernel: the device must hold
// its LDS, and its dynamic LDS size is set.
template <int D, class VF>
static int mfma_kernel_setup() {
    constexpr int NC = VF::kComputeWaves;
    using K = WsCfg<D, NC, VF>;
    auto kern = decode_attn_mfma_kernel<D, NC, VF>;
    static bool done = false;
    if (done) return SS_OK;
    int dev = 0, max_lds = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&max_lds, hipDeviceAttributeSharedMemPerBlockOptin, dev);
    if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(LDS)");
    SS_UNSUPPORTED(max_lds >= K::kLds, "decode needs %d bytes of LDS per workgroup, device has %d", K::kLds,
                   max_lds);
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            K::kLds);
    if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(decode mfma)");
    done = true;
    return SS_OK;
}

template <int D, class VF>
static int launch_mfma_kernel(DecodeCommon c, const typename VF::Args &va, const DecodeShape &s,
                              hipStream_t st) {
    constexpr int NC = VF::kComputeWaves;
    using K = WsCfg<D, NC, VF>;
    auto kern = decode_attn_mfma_kernel<D, NC, VF>;
    const int rc = mfma_kernel_setup<D, VF>();
    if (rc) return rc;
    hipLaunchKernelGGL(kern, dim3(s.S, s.n_cols), dim3(K::kWaves * kWave), K::kLds, st, c, va);
    SS_LAUNCH_CHECK("decode_attn_mfma_kernel launch");
    if (c.fused_merge) return SS_OK;  // the kernel merges its splits itself
    return launch_merge<D>(c, s, st);
}

// the format's kernel, or its heavy-dim variant when the call carries fp16
// heavy key dims
template <int D, class VF>
static int launch_mfma(DecodeCommon c, const typename VF::Args &va, const DecodeShape &s,
                       hipStream_t st) {
    if (c.nhd > 0) {
        if constexpr (VfHeavyCapable<VF>::value)
            return launch_mfma_kernel<D, WithHeavy<VF>>(c, va, s, st);
        SS_UNSUPPORTED(false, "fp16 heavy key dims are not taken by this decode shape");
    }
    return launch_mfma_kernel<D, VF>(c, va, s, st);
}

template <int NH8>
static int launch_sunv_mfma(const DecodeCommon &c, const typename VSunV<128, 4>::Args &va,
                            const DecodeShape &s, hipStream_t st) {
    auto kern = sunv_mfma_kernel<NH8>;
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 kSvLdsBytes);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(sunv mfma)");
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(s.S, s.n_cols), dim3(kSvWaves * kWave), kSvLdsBytes, st, c, va);
    SS_LAUNCH_CHECK("sunv_mfma_kernel launch");
    return SS_OK;
}

template <int D, int R, class VF>
static int launch(DecodeCommon c, const typename VF::Args &va, const DecodeShape &s,
                  hipStream_t st, bool merge = true) {
    constexpr int TH = VfThreads<VF>::value;
    const size_t lds = decode_lds_bytes<D, R, TH / kWave>() + VfLds<VF>::value;
    auto kern = decode_attn_kernel<D, R, VF>;
    static bool attr_set = false;  // per instantiation
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(decode)");
        attr_set = true;
    }
    dim3 grid(s.S, s.n_cols, VfSlabs<VF>::value);
    hipLaunchKernelGGL(kern, grid, dim3(TH), lds, st, c, va);
    SS_LAUNCH_CHECK("decode_attn_kernel launch");
    return merge ? launch_merge<D>(c, s, st) : SS_OK;
}

template <int D, class VF>
static int launch_r(DecodeCommon c, const typename VF::Args &va, const DecodeShape &s,
                    hipStream_t st, bool merge = true) {
    if (s.R == 1) return launch<D, 1, VF>(c, va, s, st, merge);
    return launch<D, 4, VF>(c, va, s, st, merge);
}

static int check_common(const void *q, int q_dtype, int64_t batch, int hq, int hkv, int64_t t_q,
                        int head_dim, const float *centroids, int n_blocks, int n_centroids,
                        const uint8_t *idx, int64_t cap, int64_t t_kv, void *out, int out_dtype) {
    SS_REQUIRE(q && centroids && idx && out, "null pointer argument");
    SS_REQUIRE(valid_dtype(q_dtype) && valid_dtype(out_dtype), "bad dtype code");
    SS_REQUIRE(batch >= 1 && hq >= 1 && hkv >= 1 && t_q >= 1, "empty batch/heads/t_q");
    SS_REQUIRE(hq % hkv == 0, "n_q_heads (%d) must be a multiple of n_kv_heads (%d)", hq, hkv);
    SS_UNSUPPORTED(head_dim == 64 || head_dim == 128,
                   "head_dim %d unsupported (64 or 128)", head_dim);
    SS_UNSUPPORTED(n_blocks * kBlockDim == head_dim,
                   "fused kernel needs block_dim 8 (n_blocks %d, head_dim %d)", n_blocks, head_dim);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256,
                   "n_centroids %d unsupported (1..256, uint8 indices)", n_centroids);
    SS_REQUIRE(t_kv >= 0 && t_kv <= cap, "t_kv %lld outside [0, cap=%lld]", (long long)t_kv,
               (long long)cap);
    SS_REQUIRE(((uintptr_t)idx % 16) == 0, "idx must be 16-byte aligned");
    SS_REQUIRE(((uintptr_t)centroids % 16) == 0, "centroids must be 16-byte aligned");
    return SS_OK;
}

// Sticky wait-failure word of this code object, one per device (kWait* bits).
__device__ unsigned int g_wait_fail_word;

// Spin limit of the bounded waits for later launches (ss_debug_set_spin_limit).
static std::atomic<int> g_spin_limit{kSpinLimit};

// Pinned host word that a give-up also stores its bits into (one per
// process, mapped into every device): the host polls it after the fact
// with a plain load, so the check costs no synchronisation.
static int wait_host_word(unsigned int **host, unsigned int **dev_ptr) {
    static std::mutex mu;
    static unsigned int *h = nullptr, *d = nullptr;
    std::lock_guard<std::mutex> lock(mu);
    if (!h) {
        void *p = nullptr;
        hipError_t e = hipHostMalloc(&p, 64, hipHostMallocPortable | hipHostMallocMapped |
                                                 hipHostMallocCoherent);
        if (e != hipSuccess) return hip_fail(e, "hipHostMalloc(wait flag)");
        void *dp = nullptr;
        e = hipHostGetDevicePointer(&dp, p, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(p);
            return hip_fail(e, "hipHostGetDevicePointer(wait flag)");
        }
        h = static_cast<unsigned int *>(p);
        *h = 0u;
        d = static_cast<unsigned int *>(dp);
    }
    if (host) *host = h;
    if (dev_ptr) *dev_ptr = d;
    return SS_OK;
}

// Device address of g_wait_fail_word on the current device, looked up once
// per device.
static int wait_word(unsigned int **out) {
    static std::mutex mu;
    static unsigned int *addr[64] = {nullptr};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    SS_UNSUPPORTED(dev >= 0 && dev < 64, "device ordinal %d beyond 63", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_wait_fail_word));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(wait word)");
        addr[dev] = static_cast<unsigned int *>(p);
    }
    *out = addr[dev];
    return SS_OK;
}

static int fill_common(DecodeCommon &c, const DecodeShape &s, const void *q, int q_dtype,
                       int hq, int hkv, int64_t t_q, float scale, const int32_t *perm,
                       const float *centroids, int n_centroids, const uint8_t *idx, int64_t cap,
                       int64_t t_kv, int causal, int64_t q_offset, void *out, int out_dtype,
                       void *ws, size_t ws_bytes, int head_dim) {
    c.q = q;
    c.perm = perm;
    c.centroids = centroids;
    c.idx = idx;
    c.out = out;
    c.q_dtype = q_dtype;
    c.out_dtype = out_dtype;
    c.n_q_heads = hq;
    c.n_kv_heads = hkv;
    c.rep = hq / hkv;
    c.n_rg = s.n_rg;
    c.t_q = t_q;
    c.rows_total = (int64_t)c.rep * t_q;
    c.n_centroids = n_centroids;
    c.cap = cap;
    c.t_kv = t_kv;
    c.scale = scale;
    c.causal = causal ? 1 : 0;
    c.q_offset = q_offset;
    c.n_splits = s.S;
    c.tiles_per_split = s.tiles_per_split;
    c.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
    {
        int rc = wait_word(&c.wait_fail);
        if (rc == SS_OK) rc = wait_host_word(nullptr, &c.wait_host);
        if (rc != SS_OK) return rc;
    }
    c.kheavy = nullptr;
    c.heavy_dims = nullptr;
    c.nhd = 0;
    c.rot = nullptr;
    c.part_ml = nullptr;
    c.part_acc = nullptr;
    c.part_cnt = nullptr;
    c.fused_merge = s.S > 1 && (size_t)s.n_cols * sizeof(int) <= kCntBytes;
    // columns' counters up to 4 KiB apart, so the splits of different
    // columns never contend for one cache line
    c.cnt_stride = 1024;
    while (c.cnt_stride > 1 && (size_t)s.n_cols * c.cnt_stride * sizeof(int) > kCntBytes)
        c.cnt_stride /= 2;
    if (s.S > 1) {
        const size_t need = decode_ws_bytes(s, head_dim);
        if (!ws || ws_bytes < need) {
            set_error("decode workspace too small: need %zu bytes, got %zu", need,
                      ws ? ws_bytes : (size_t)0);
            return SS_ERR_WORKSPACE;
        }
        SS_REQUIRE(((uintptr_t)ws % 256) == 0, "workspace must be 256-byte aligned");
        const WsLayout w = ws_layout(s, head_dim);
        char *base = reinterpret_cast<char *>(ws);
        c.part_cnt = reinterpret_cast<int *>(base + w.cnt);
        c.part_ml = reinterpret_cast<float *>(base + w.ml);
        c.part_acc = reinterpret_cast<float *>(base + w.acc);
    }
    return SS_OK;
}

}  // namespace ss

using namespace ss;

extern "C" int ss_decode_wait_failures(void *stream, int clear, unsigned int *flags) {
    unsigned int *w = nullptr;
    int rc = wait_word(&w);
    if (rc != SS_OK) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    unsigned int v = 0;
    e = hipMemcpy(&v, w, sizeof(v), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "hipMemcpy(wait word)");
    unsigned int *hw = nullptr;
    rc = wait_host_word(&hw, nullptr);
    if (rc != SS_OK) return rc;
    v |= __atomic_load_n(hw, __ATOMIC_ACQUIRE);
    if (flags) *flags = v;
    if (v && clear) {
        const unsigned int zero = 0;
        e = hipMemcpy(w, &zero, sizeof(zero), hipMemcpyHostToDevice);
        if (e != hipSuccess) return hip_fail(e, "hipMemcpy(clear wait word)");
        __atomic_store_n(hw, 0u, __ATOMIC_RELEASE);
    }
    if (v) {
        set_error("a bounded wait of a fused decode gave up (flags 0x%x: %s%s%s); the output of "
                  "that launch is invalid", v, (v & kWaitBarrier) ? "compute barrier " : "",
                  (v & kWaitSlot) ? "ring slot " : "", (v & kWaitTile) ? "ring tile" : "");
        return SS_ERR_WAIT;
    }
    return SS_OK;
}

extern "C" int ss_decode_wait_flag_host(unsigned int **flag) {
    SS_REQUIRE(flag, "null pointer argument");
    return wait_host_word(flag, nullptr);
}

extern "C" int ss_debug_set_spin_limit(int limit) {
    g_spin_limit.store(limit < 0 ? kSpinLimit : limit, std::memory_order_relaxed);
    return SS_OK;
}

extern "C" size_t ss_decode_workspace_bytes(int64_t batch, int n_q_heads, int n_kv_heads,
                                            int64_t t_q, int head_dim, int64_t t_kv,
                                            int n_splits) {
    if (batch < 1 || n_q_heads < 1 || n_kv_heads < 1 || n_q_heads % n_kv_heads || t_q < 1)
        return 0;
    return decode_ws_bytes(decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits),
                           head_dim);
}

extern "C" int ss_decode_default_splits(int64_t batch, int n_q_heads, int n_kv_heads,
                                        int64_t t_q, int head_dim, int64_t t_kv) {
    (void)head_dim;
    if (batch < 1 || n_q_heads < 1 || n_kv_heads < 1 || n_q_heads % n_kv_heads || t_q < 1)
        return 0;
    return decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, 0).S;
}

static int dense_checks(const void *values, int v_dtype) {
    SS_REQUIRE(values, "null values");
    SS_REQUIRE(valid_dtype(v_dtype), "bad value dtype");
    SS_REQUIRE(((uintptr_t)values % 16) == 0, "values must be 16-byte aligned");
    return SS_OK;
}

// The VALU decode over dense values (merge: whether it launches its own merge).
static int launch_dense(const DecodeCommon &c, const DecodeShape &s, hipStream_t st, int head_dim,
                        const void *values, int v_dtype, bool merge) {
#define SS_DENSE(DD, TT)                                                                  \
    {                                                                                     \
        typename VDense<DD, TT>::Args va{reinterpret_cast<const TT *>(values)};           \
        return launch_r<DD, VDense<DD, TT>>(c, va, s, st, merge);                         \
    }
    if (head_dim == 128) {
        if (v_dtype == SS_F16) SS_DENSE(128, __half)
        if (v_dtype == SS_BF16) SS_DENSE(128, __hip_bfloat16)
        SS_DENSE(128, float)
    } else {
        if (v_dtype == SS_F16) SS_DENSE(64, __half)
        if (v_dtype == SS_BF16) SS_DENSE(64, __hip_bfloat16)
        SS_DENSE(64, float)
    }
#undef SS_DENSE
}

extern "C" int ss_decode_attn_dense(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                    int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                    const int32_t *perm, const float *centroids, int n_blocks,
                                    int n_centroids, const uint8_t *idx, const void *values,
                                    int v_dtype, int64_t cap, int64_t t_kv, int causal,
                                    int64_t q_offset, void *out, int out_dtype, void *workspace,
                                    size_t workspace_bytes, int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    if ((rc = dense_checks(values, v_dtype))) return rc;
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits);
    DecodeCommon c;
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, centroids,
                     n_centroids, idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    return launch_dense(c, s, reinterpret_cast<hipStream_t>(stream), head_dim, values, v_dtype,
                        true);
}

static int grouped_checks(int head_dim, const uint32_t *packed, const void *scales,
                          const void *zeros, int sz_dtype, int bits, int group_size) {
    SS_REQUIRE(packed && scales && zeros, "null packed/scales/zeros");
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4 (got %d)", bits);
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(group_size >= 1 && head_dim % group_size == 0,
               "head_dim %d not divisible by group_size %d", head_dim, group_size);
    SS_REQUIRE(!(bits == 2 && head_dim % 16) && !(bits == 4 && head_dim % 8),
               "head_dim %d cannot be packed at %d bits", head_dim, bits);
    // a packed word spans at most two scale groups
    SS_UNSUPPORTED(group_size >= 32 / bits, "group_size %d < %d values per word", group_size,
                   32 / bits);
    SS_REQUIRE(((uintptr_t)packed % 4) == 0, "packed values must be 4-byte aligned");
    return SS_OK;
}

// The VALU decode over reference-format grouped values (merge: whether it
// launches its own merge).
static int launch_grouped(const DecodeCommon &c, const DecodeShape &s, hipStream_t st,
                          int head_dim, const uint32_t *packed, const void *scales,
                          const void *zeros, int sz_dtype, int bits, int group_size, bool merge) {
    const int n_groups = head_dim / group_size;
#define SS_GROUPED(DD, BB, SZT)                                                          \
    {                                                                                    \
        typename VGrouped<DD, BB, SZT>::Args va{packed, reinterpret_cast<const SZT *>(scales), \
                                                reinterpret_cast<const SZT *>(zeros),    \
                                                group_size, n_groups};                   \
        return launch_r<DD, VGrouped<DD, BB, SZT>>(c, va, s, st, merge);                 \
    }
#define SS_GROUPED_BITS(DD, SZT)            \
    {                                       \
        if (bits == 2) SS_GROUPED(DD, 2, SZT) \
        if (bits == 3) SS_GROUPED(DD, 3, SZT) \
        SS_GROUPED(DD, 4, SZT)              \
    }
    if (head_dim == 128) {
        if (sz_dtype == SS_F16) SS_GROUPED_BITS(128, __half)
        SS_GROUPED_BITS(128, float)
    } else {
        if (sz_dtype == SS_F16) SS_GROUPED_BITS(64, __half)
        SS_GROUPED_BITS(64, float)
    }
#undef SS_GROUPED_BITS
#undef SS_GROUPED
}

extern "C" int ss_decode_attn_grouped(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                      int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                      const int32_t *perm, const float *centroids, int n_blocks,
                                      int n_centroids, const uint8_t *idx,
                                      const uint32_t *packed, const void *scales,
                                      const void *zeros, int sz_dtype, int bits,
                                      int group_size, int64_t cap, int64_t t_kv, int causal,
                                      int64_t q_offset, void *out, int out_dtype, void *workspace,
                                      size_t workspace_bytes, int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    if ((rc = grouped_checks(head_dim, packed, scales, zeros, sz_dtype, bits, group_size)))
        return rc;
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits);
    DecodeCommon c;
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, centroids,
                     n_centroids, idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    return launch_grouped(c, s, reinterpret_cast<hipStream_t>(stream), head_dim, packed, scales,
                          zeros, sz_dtype, bits, group_size, true);
}

// Workspace of the TurboQuant decode: the split partials (as for the other
// VALU decodes, plus one slot per column for buffered tokens), then the fp32
// output rows of the rotated basis.
static DecodeShape with_buffer_slot(DecodeShape s, int64_t t_buf) {
    if (t_buf > 0) s.S += 1;
    return s;
}

static size_t turboquant_ws_bytes(const DecodeShape &sw, int64_t rows, int head_dim) {
    // the rows never overlap the split counters at the workspace's start,
    // which the matrix-core decodes sharing this workspace rely on being zero
    // (with one split there are no partials, but the counter area stays)
    size_t part = decode_ws_bytes(sw, head_dim);
    if (part < kCntBytes) part = kCntBytes;
    part = (part + 255) / 256 * 256;
    return part + (size_t)rows * head_dim * sizeof(float);
}

extern "C" size_t ss_decode_turboquant_workspace_bytes(int64_t batch, int n_q_heads,
                                                       int n_kv_heads, int64_t t_q, int head_dim,
                                                       int64_t t_kv, int64_t t_buf, int n_splits) {
    if (batch < 1 || n_q_heads < 1 || n_kv_heads < 1 || n_q_heads % n_kv_heads || t_q < 1)
        return 0;
    // enough for every split policy of the transformed-basis decodes (the
    // VALU kernel's, the matrix-core TurboQuant and SunShape-value kernels')
    size_t need = 0;
    for (int kind : {kKindValu, kKindMfma, kKindSunv}) {
        const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits, kind);
        need = std::max(need, turboquant_ws_bytes(with_buffer_slot(s, t_buf), batch * n_q_heads * t_q,
                                                  head_dim));
    }
    return need;
}

// Shared host side of the decodes whose values accumulate in a transformed
// basis (TurboQuant's rotation, a SunShape value codec's permutation or
// rotation): the VALU decode writes y (fp32, that basis) or split partials;
// buffered original-basis tokens become one more partial, taken into that
// basis with transform^T (orthogonal); the merge launch, or rotate_rows_kernel
// for a single split, writes out = y @ transform in out_dtype.  A null
// transform is the identity (values in the original basis: the grouped and
// dense VALU decodes with a hybrid cache's buffer): the kernels and the merge
// write out directly.
template <class MainLaunch>
static int transformed_decode(const void *q, int q_dtype, int64_t batch, int hq, int hkv,
                              int64_t t_q, int head_dim, float scale, const int32_t *perm,
                              const float *centroids, int n_centroids, const uint8_t *idx,
                              int64_t cap, int64_t t_kv, const float *transform,
                              const void *k_buf, const void *v_buf, int buf_dtype,
                              int64_t buf_sb, int64_t buf_sh, int64_t buf_st, int64_t t_buf,
                              int causal, int64_t q_offset, void *out, int out_dtype,
                              void *workspace, size_t workspace_bytes, int n_splits,
                              void *stream, MainLaunch &&launch_main, int kind = kKindValu) {
    const bool ident = transform == nullptr;
    SS_REQUIRE(((uintptr_t)transform % 4) == 0, "misaligned transform/rotation matrix");
    SS_REQUIRE(t_buf >= 0, "negative buffer length");
    if (t_buf > 0) {
        SS_REQUIRE(k_buf && v_buf, "null buffer keys/values");
        SS_REQUIRE(buf_dtype == SS_F16 || buf_dtype == SS_BF16 || buf_dtype == SS_F32,
                   "buffer dtype must be f16, bf16 or f32");
        SS_REQUIRE(buf_sb >= 0 && buf_sh >= 0 && buf_st >= head_dim,
                   "buffer strides must be non-negative, token stride >= head_dim");
    }
    const DecodeShape s = decode_shape(batch, hq, hkv, t_q, t_kv, n_splits, kind);
    const DecodeShape sw = with_buffer_slot(s, t_buf);  // partial slots incl. the buffer's
    const int64_t rows = batch * hq * t_q;
    const size_t need = turboquant_ws_bytes(sw, rows, head_dim);
    if (!workspace || workspace_bytes < need) {
        set_error("decode workspace too small: need %zu bytes, got %zu", need,
                  workspace ? workspace_bytes : (size_t)0);
        return SS_ERR_WORKSPACE;
    }
    SS_REQUIRE(((uintptr_t)workspace % 256) == 0, "workspace must be 256-byte aligned");
    float *y = reinterpret_cast<float *>(static_cast<char *>(workspace) + need -
                                         (size_t)rows * head_dim * sizeof(float));
    DecodeCommon c;
    int rc = fill_common(c, sw, q, q_dtype, hq, hkv, t_q, scale, perm, centroids, n_centroids,
                         idx, cap, t_kv, causal, q_offset, ident ? out : y,
                         ident ? out_dtype : SS_F32, workspace, workspace_bytes, head_dim);
    if (rc) return rc;
    c.tiles_per_split = s.tiles_per_split;  // the compressed tokens' splits: grid s.S
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    rc = launch_main(c, s, st);  // no merge: it follows the buffer's partial
    if (rc) return rc;
    if (t_buf > 0) {
#define SS_BUFP(DD, RR)                                                                       \
    hipLaunchKernelGGL((buffer_partial_kernel<DD, RR>), dim3(sw.n_cols), dim3(256), 0, st, c,   \
                       k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, t_buf, transform, s.S)
        if (head_dim == 128) {
            if (sw.R == 1) SS_BUFP(128, 1); else SS_BUFP(128, 4);
        } else {
            if (sw.R == 1) SS_BUFP(64, 1); else SS_BUFP(64, 4);
        }
#undef SS_BUFP
        SS_LAUNCH_CHECK("buffer_partial_kernel launch");
    }
    if (sw.S > 1)
        return head_dim == 128 ? launch_merge<128>(c, sw, st, transform, out, out_dtype)
                               : launch_merge<64>(c, sw, st, transform, out, out_dtype);
    if (ident) return SS_OK;  // the one split wrote out
    const unsigned blocks = (unsigned)((rows + kRotRows - 1) / kRotRows);
    if (head_dim == 128)
        hipLaunchKernelGGL(rotate_rows_kernel<128>, dim3(blocks), dim3(256), 0, st, y, transform,
                           rows, out, out_dtype);
    else
        hipLaunchKernelGGL(rotate_rows_kernel<64>, dim3(blocks), dim3(256), 0, st, y, transform,
                           rows, out, out_dtype);
    SS_LAUNCH_CHECK("rotate_rows_kernel launch");
    return SS_OK;
}

extern "C" int ss_decode_attn_turboquant(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint32_t *packed, const float *norms,
    const float *levels, const float *rotation, int bits, int64_t cap, int64_t t_kv,
    const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
    int64_t buf_st, int64_t t_buf, const void *k_heavy, const int32_t *heavy_dims, int n_heavy_dims,
    int causal, int64_t q_offset, void *out, int out_dtype, void *workspace, size_t workspace_bytes,
    int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(packed && norms && levels && rotation, "null packed/norms/levels/rotation");
    if (k_heavy) {
        SS_REQUIRE(heavy_dims, "null heavy_dims");
        SS_UNSUPPORTED(n_heavy_dims > 0 && n_heavy_dims % 8 == 0 && n_heavy_dims <= 64,
                       "n_heavy_dims %d unsupported (a positive multiple of 8, at most 64)",
                       n_heavy_dims);
        SS_REQUIRE(((uintptr_t)k_heavy % 16) == 0, "heavy keys must be 16-byte aligned");
    }
    SS_REQUIRE(bits == 2 || bits == 3 || bits == 4, "bits must be 2, 3 or 4 (got %d)", bits);
    SS_REQUIRE(!(bits == 2 && head_dim % 16) && !(bits == 4 && head_dim % 8),
               "head_dim %d cannot be packed at %d bits", head_dim, bits);
    SS_REQUIRE(((uintptr_t)packed % 4) == 0 && ((uintptr_t)norms % 4) == 0,
               "packed/norms must be 4-byte aligned");
    auto main = [&](const DecodeCommon &c, const DecodeShape &s, hipStream_t st) -> int {
#define SS_TURBO(DD, BB)                                                    \
    {                                                                       \
        typename VTurbo<DD, BB>::Args va{packed, norms, {},                 \
                                         static_cast<const __half *>(k_heavy), \
                                         heavy_dims, k_heavy ? n_heavy_dims : 0}; \
        for (int i = 0; i < (1 << BB); ++i) va.lv[i] = levels[i];           \
        return launch_r<DD, VTurbo<DD, BB>>(c, va, s, st, false);           \
    }
        if (head_dim == 128) {
            if (bits == 2) SS_TURBO(128, 2)
            if (bits == 3) SS_TURBO(128, 3)
            SS_TURBO(128, 4)
        }
        if (bits == 2) SS_TURBO(64, 2)
        if (bits == 3) SS_TURBO(64, 3)
        SS_TURBO(64, 4)
#undef SS_TURBO
    };
    return transformed_decode(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                              centroids, n_centroids, idx, cap, t_kv, rotation, k_buf, v_buf,
                              buf_dtype, buf_sb, buf_sh, buf_st, t_buf, causal, q_offset, out,
                              out_dtype, workspace, workspace_bytes, n_splits, stream, main);
}

extern "C" int ss_decode_attn_grouped_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint32_t *packed, const void *scales,
    const void *zeros, int sz_dtype, int bits, int group_size, int64_t cap, int64_t t_kv,
    const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
    int64_t buf_st, int64_t t_buf, int causal, int64_t q_offset, void *out, int out_dtype,
    void *workspace, size_t workspace_bytes, int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    if ((rc = grouped_checks(head_dim, packed, scales, zeros, sz_dtype, bits, group_size)))
        return rc;
    auto main = [&](const DecodeCommon &c, const DecodeShape &s, hipStream_t st) -> int {
        return launch_grouped(c, s, st, head_dim, packed, scales, zeros, sz_dtype, bits,
                              group_size, false);
    };
    return transformed_decode(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                              centroids, n_centroids, idx, cap, t_kv, nullptr, k_buf, v_buf,
                              buf_dtype, buf_sb, buf_sh, buf_st, t_buf, causal, q_offset, out,
                              out_dtype, workspace, workspace_bytes, n_splits, stream, main);
}

extern "C" int ss_decode_attn_dense_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const void *values, int v_dtype, int64_t cap,
    int64_t t_kv, const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb,
    int64_t buf_sh, int64_t buf_st, int64_t t_buf, int causal, int64_t q_offset, void *out,
    int out_dtype, void *workspace, size_t workspace_bytes, int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    if ((rc = dense_checks(values, v_dtype))) return rc;
    auto main = [&](const DecodeCommon &c, const DecodeShape &s, hipStream_t st) -> int {
        return launch_dense(c, s, st, head_dim, values, v_dtype, false);
    };
    return transformed_decode(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                              centroids, n_centroids, idx, cap, t_kv, nullptr, k_buf, v_buf,
                              buf_dtype, buf_sb, buf_sh, buf_st, t_buf, causal, q_offset, out,
                              out_dtype, workspace, workspace_bytes, n_splits, stream, main);
}

extern "C" int ss_decode_attn_sunshape_v(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const float *centroids, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint8_t *v_idx, const float *v_centroids,
    int v_block_dim, int v_n_centroids, const float *v_transform, const void *k_heavy,
    const int32_t *heavy_dims, int n_heavy_dims, int64_t cap, int64_t t_kv,
    const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
    int64_t buf_st, int64_t t_buf, int causal, int64_t q_offset, void *out, int out_dtype,
    void *workspace, size_t workspace_bytes, int n_splits, void *stream) {
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(v_idx && v_centroids, "null value indices/centroids");
    SS_UNSUPPORTED(v_block_dim == 4 || v_block_dim == 8, "value block_dim %d unsupported (4 or 8)",
                   v_block_dim);
    SS_UNSUPPORTED(v_n_centroids >= 1 && v_n_centroids <= 256,
                   "value n_centroids %d unsupported (1..256, uint8 indices)", v_n_centroids);
    SS_REQUIRE(((uintptr_t)v_idx % 4) == 0, "value indices must be 4-byte aligned");
    SS_REQUIRE(((uintptr_t)v_centroids % 16) == 0, "value centroids must be 16-byte aligned");
    if (k_heavy) {
        SS_REQUIRE(heavy_dims, "null heavy_dims");
        SS_UNSUPPORTED(n_heavy_dims > 0 && n_heavy_dims % 8 == 0 && n_heavy_dims <= 64,
                       "n_heavy_dims %d unsupported (a positive multiple of 8, at most 64)",
                       n_heavy_dims);
        SS_REQUIRE(((uintptr_t)k_heavy % 16) == 0, "heavy keys must be 16-byte aligned");
    }
    // the matrix-core kernel: head_dim 128, value block_dim 4, four query
    // rows per column, 0/8/16/32/64 heavy dims, 8-byte aligned value indices
    const int nh8 = k_heavy ? n_heavy_dims / 8 : 0;
    const bool sv_mfma = head_dim == 128 && v_block_dim == 4 && ((uintptr_t)v_idx % 8) == 0 &&
                         cap < (int64_t(1) << 26) &&
                         (nh8 == 0 || nh8 == 1 || nh8 == 2 || nh8 == 4 || nh8 == 8);
    auto main = [&](const DecodeCommon &c, const DecodeShape &s, hipStream_t st) -> int {
        if (sv_mfma && s.R == kMfmaRows) {
            const typename VSunV<128, 4>::Args va{v_idx, v_centroids, v_n_centroids,
                                                  static_cast<const __half *>(k_heavy),
                                                  heavy_dims, k_heavy ? n_heavy_dims : 0};
            switch (nh8) {
                case 1: return launch_sunv_mfma<1>(c, va, s, st);
                case 2: return launch_sunv_mfma<2>(c, va, s, st);
                case 4: return launch_sunv_mfma<4>(c, va, s, st);
                case 8: return launch_sunv_mfma<8>(c, va, s, st);
                default: return launch_sunv_mfma<0>(c, va, s, st);
            }
        }
#define SS_SUNV(DD, BB)                                                     \
    {                                                                       \
        typename VSunV<DD, BB>::Args va{v_idx, v_centroids, v_n_centroids,    \
                                        static_cast<const __half *>(k_heavy), \
                                        heavy_dims, k_heavy ? n_heavy_dims : 0}; \
        return launch_r<DD, VSunV<DD, BB>>(c, va, s, st, false);            \
    }
        if (head_dim == 128) {
            if (v_block_dim == 4) SS_SUNV(128, 4)
            SS_SUNV(128, 8)
        }
        if (v_block_dim == 4) SS_SUNV(64, 4)
        SS_SUNV(64, 8)
#undef SS_SUNV
    };
    // the matrix-core kernel's split policy asks no more splits (and so no
    // more workspace) than the VALU one ss_decode_turboquant_workspace_bytes
    // sizes for
    return transformed_decode(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                              centroids, n_centroids, idx, cap, t_kv, v_transform, k_buf, v_buf,
                              buf_dtype, buf_sb, buf_sh, buf_st, t_buf, causal, q_offset, out,
                              out_dtype, workspace, workspace_bytes, n_splits, stream, main,
                              sv_mfma ? kKindSunv : kKindValu);
}

extern "C" int ss_decode_plan(int kind, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
                              int head_dim, int64_t t_kv, int n_splits, int *splits_out,
                              size_t *workspace_bytes_out) {
    SS_REQUIRE(kind == kKindValu || kind == kKindMfma, "kind must be 0 (dense) or 1 (il8)");
    SS_REQUIRE(batch >= 1 && n_q_heads >= 1 && n_kv_heads >= 1 && t_q >= 1 &&
                   n_q_heads % n_kv_heads == 0,
               "bad head/batch counts");
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits, kind);
    if (splits_out) *splits_out = s.S;
    if (workspace_bytes_out) *workspace_bytes_out = decode_ws_bytes(s, head_dim);
    return SS_OK;
}

// Tiles of the prepared codebook: 16 centroids of 4 consecutive blocks.
__host__ __device__ inline int cb_tiles(int n_blocks, int n_centroids) {
    return (n_blocks / 4) * ((n_centroids + 15) / 16);
}

// One workgroup: max |C| over the codebook, then C' = C * 2^(kCbMaxExp - e)
// (max |C| < 2^e) split into fp16 hi/lo, stored in the order the LUT build's
// matrix-core operands are loaded: tile (bg, ct) of 4 blocks x 16 centroids
// holds 64 lanes x 8 halves for hi, then the same for lo, where lane l
// carries centroid ct*16 + l%16 of block bg*4 + l/16 (zero past the last
// centroid).  The multiplier 2^(e - kCbMaxExp) that undoes the scale follows
// as a float.
__global__ void __launch_bounds__(1024) codebook_f16x2_kernel(const float *cents, int n_blocks,
                                                              int n_centroids, _Float16 *out) {
    __shared__ float red[1024 / kWave];
    const int n = n_blocks * n_centroids * kBlockDim;
    float mx = 0.f;
    for (int i = threadIdx.x; i < n; i += 1024) mx = fmaxf(mx, fabsf(cents[i]));
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < 1024 / kWave; ++w) mx = fmaxf(mx, red[w]);
    int ex = 0;
    frexpf(mx, &ex);  // mx < 2^ex
    const int sh = kCbMaxExp - ex;
    const int nct = (n_centroids + 15) / 16;
    const int n_lanes = cb_tiles(n_blocks, n_centroids) * kWave;
    for (int i = threadIdx.x; i < n_lanes * kBlockDim; i += 1024) {
        const int j = i % kBlockDim, lane = (i / kBlockDim) % kWave, tile = i / (kBlockDim * kWave);
        const int bg = tile / nct, ct = tile % nct;
        const int b = bg * 4 + lane / 16, cc = ct * 16 + lane % 16;
        const float v = cc < n_centroids
                            ? ldexpf(cents[((int64_t)b * n_centroids + cc) * kBlockDim + j], sh)
                            : 0.f;
        const _Float16 hi = (_Float16)v;
        _Float16 *o = out + (int64_t)tile * 2 * kWave * kBlockDim + lane * kBlockDim + j;
        o[0] = hi;
        o[kWave * kBlockDim] = (_Float16)((v - (float)hi) * kSplitScale);
    }
    if (threadIdx.x == 0)
        *reinterpret_cast<float *>(out + (int64_t)n_lanes * 2 * kBlockDim) = ldexpf(1.f, -sh);
    // |C|^2 of each lane's centroid (unscaled float32, 0 past the last
    // centroid), in the tiles' lane order, after the scale's 16 bytes
    float *nrm = reinterpret_cast<float *>(out + (int64_t)n_lanes * 2 * kBlockDim) + 4;
    for (int i = threadIdx.x; i < n_lanes; i += 1024) {
        const int lane = i % kWave, tile = i / kWave;
        const int bg = tile / nct, ct = tile % nct;
        const int b = bg * 4 + lane / 16, cc = ct * 16 + lane % 16;
        float acc = 0.f;
        if (cc < n_centroids)
            for (int j = 0; j < kBlockDim; ++j) {
                const float x = cents[((int64_t)b * n_centroids + cc) * kBlockDim + j];
                acc = fmaf(x, x, acc);
            }
        nrm[i] = acc;
    }
}

extern "C" size_t ss_codebook_f16x2_bytes(int n_blocks, int n_centroids) {
    if (n_blocks < 4 || n_blocks % 4 || n_centroids < 1) return 0;
    return (size_t)cb_tiles(n_blocks, n_centroids) * kWave * (2 * 16 + 4) + 16;
}

extern "C" int ss_codebook_f16x2(const float *centroids, int n_blocks, int n_centroids,
                                 void *out, void *stream) {
    SS_REQUIRE(centroids && out, "null centroids/out");
    SS_REQUIRE(n_blocks >= 4 && n_blocks <= 64 && n_blocks % 4 == 0 && n_centroids >= 1 &&
                   n_centroids <= kLutStride,
               "bad codebook shape (%d blocks, %d centroids)", n_blocks, n_centroids);
    SS_REQUIRE(((uintptr_t)out % 16) == 0, "prepared codebook must be 16-byte aligned");
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(codebook_f16x2_kernel, dim3(1), dim3(1024), 0, st, centroids, n_blocks,
                       n_centroids, static_cast<_Float16 *>(out));
    SS_LAUNCH_CHECK("codebook_f16x2_kernel launch");
    return SS_OK;
}

// Checks shared by the hybrid entry points: t_buf buffered tokens at k_buf /
// v_buf with element strides buf_sb, buf_sh, buf_st.
static int check_buffer(const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb,
                        int64_t buf_sh, int64_t buf_st, int64_t t_buf, int head_dim) {
    SS_REQUIRE(t_buf >= 0, "negative buffer length");
    if (t_buf == 0) return SS_OK;
    SS_REQUIRE(k_buf && v_buf, "null buffer keys/values");
    SS_REQUIRE(buf_dtype == SS_F16 || buf_dtype == SS_BF16 || buf_dtype == SS_F32,
               "buffer dtype must be f16, bf16 or f32");
    SS_REQUIRE(buf_sb >= 0 && buf_sh >= 0 && buf_st >= head_dim,
               "buffer strides must be non-negative, token stride >= head_dim");
    SS_REQUIRE(((uintptr_t)k_buf % 16) == 0 && buf_sb % 8 == 0 && buf_sh % 8 == 0 &&
                   buf_st % 8 == 0,
               "buffer keys must be 16-byte aligned with strides a multiple of 8 elements");
    return SS_OK;
}

// fp16 heavy-block key dims of a mixed-precision codec for the matrix-core
// kernels (hybrid caches): [rows][n] halves at 16-byte aligned rows.
static int set_heavy(DecodeCommon &c, const void *k_heavy, const int32_t *heavy_dims, int n) {
    if (!k_heavy) return SS_OK;
    SS_REQUIRE(heavy_dims, "null heavy_dims");
    SS_UNSUPPORTED(n > 0 && n % 8 == 0 && n <= kMaxHeavyMfma,
                   "n_heavy_dims %d unsupported (a positive multiple of 8, at most %d)", n,
                   kMaxHeavyMfma);
    SS_REQUIRE(((uintptr_t)k_heavy % 16) == 0, "heavy keys must be 16-byte aligned");
    c.kheavy = static_cast<const __half *>(k_heavy);
    c.heavy_dims = heavy_dims;
    c.nhd = n;
    return SS_OK;
}

static int il8_impl(const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads,
                    int64_t t_q, int head_dim, float scale, const int32_t *perm,
                    const void *codebook, int n_blocks, int n_centroids, const uint8_t *idx,
                    const void *values_il8, int v_dtype, int64_t cap, int64_t t_kv, int causal,
                    int64_t q_offset, void *out, int out_dtype, void *workspace,
                    size_t workspace_bytes, int n_splits, const void *k_buf, const void *v_buf,
                    int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st,
                    int64_t t_buf, void *stream, const void *k_heavy = nullptr,
                    const int32_t *heavy_dims = nullptr, int n_heavy_dims = 0) {
    const float *cents = static_cast<const float *>(codebook);
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, cents,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0, "prepared codebook must be 16-byte aligned");
    SS_REQUIRE(values_il8, "null values");
    SS_UNSUPPORTED(v_dtype == SS_F16, "interleaved values must be float16");
    SS_REQUIRE(cap % 8 == 0, "cap must be a multiple of 8 for interleaved values");
    SS_REQUIRE(((uintptr_t)values_il8 % 16) == 0, "values must be 16-byte aligned");
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits,
                                       kKindMfma);
    DecodeCommon c;
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, cents,
                     n_centroids, idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    c.centroids = nullptr;
    c.codebook = static_cast<const uint4 *>(codebook);
    c.codebook_mul = reinterpret_cast<const float *>(
        static_cast<const char *>(codebook) + (size_t)cb_tiles(n_blocks, n_centroids) * 2 * kWave * 16);
    rc = check_buffer(k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, t_buf, head_dim);
    if (rc) return rc;
    rc = set_heavy(c, k_heavy, heavy_dims, n_heavy_dims);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const __half *v8 = reinterpret_cast<const __half *>(values_il8);
    if (t_buf > 0 || c.nhd > 0) {  // the hybrid cache's kernel (buffer share, heavy dims)
        if (head_dim == 128)
            return launch_mfma<128, VIl8Hyb<128>>(
                c, VIl8Hyb<128>::Args{v8, k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, t_buf},
                s, st);
        return launch_mfma<64, VIl8Hyb<64>>(
            c, VIl8Hyb<64>::Args{v8, k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, t_buf}, s,
            st);
    }
    if (head_dim == 128) return launch_mfma<128, VIl8<128>>(c, VIl8<128>::Args{v8}, s, st);
    return launch_mfma<64, VIl8<64>>(c, VIl8<64>::Args{v8}, s, st);
}

extern "C" int ss_decode_attn_il8(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                  int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                  const int32_t *perm, const void *codebook, int n_blocks,
                                  int n_centroids, const uint8_t *idx, const void *values_il8,
                                  int v_dtype, int64_t cap, int64_t t_kv, int causal,
                                  int64_t q_offset, void *out, int out_dtype, void *workspace,
                                  size_t workspace_bytes, int n_splits, void *stream) {
    return il8_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                    codebook, n_blocks, n_centroids, idx, values_il8, v_dtype, cap, t_kv, causal,
                    q_offset, out, out_dtype, workspace, workspace_bytes, n_splits, nullptr,
                    nullptr, SS_F16, 0, 0, 0, 0, stream);
}

extern "C" int ss_decode_attn_il8_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, int n_blocks,
    int n_centroids, const uint8_t *idx, const void *values_il8, int v_dtype, int64_t cap,
    int64_t t_kv, const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb,
    int64_t buf_sh, int64_t buf_st, int64_t t_buf, const void *k_heavy, const int32_t *heavy_dims,
    int n_heavy_dims, int causal, int64_t q_offset, void *out, int out_dtype, void *workspace,
    size_t workspace_bytes, int n_splits, void *stream) {
    return il8_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                    codebook, n_blocks, n_centroids, idx, values_il8, v_dtype, cap, t_kv, causal,
                    q_offset, out, out_dtype, workspace, workspace_bytes, n_splits, k_buf, v_buf,
                    buf_dtype, buf_sb, buf_sh, buf_st, t_buf, stream, k_heavy, heavy_dims,
                    n_heavy_dims);
}

extern "C" int ss_decode_step_il8(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, const float *centroids,
    int n_blocks, int n_centroids, uint8_t *idx, void *values_il8, int64_t cap, int64_t t_cache,
    const void *k_new, const void *v_new, int kv_dtype, int64_t kv_sb, int64_t kv_sh, int64_t kv_st,
    int64_t n_new, int causal, int64_t q_offset, void *out, int out_dtype, void *workspace,
    size_t workspace_bytes, int n_splits, void *stream) {
    SS_UNSUPPORTED(n_new >= 1 && n_new <= kMaxStepTokens, "a fused step takes 1..%d new tokens",
                   kMaxStepTokens);
    SS_REQUIRE(t_cache >= 1, "a fused step needs a non-empty cache (t_cache %lld)",
               (long long)t_cache);
    SS_REQUIRE(t_cache + n_new <= cap, "new tokens [%lld, %lld) past cap %lld", (long long)t_cache,
               (long long)(t_cache + n_new), (long long)cap);
    SS_UNSUPPORTED(kv_dtype == SS_F16, "a fused step takes float16 keys and values");
    SS_REQUIRE(k_new && v_new && centroids, "null new keys, values or centroids");
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256 && n_blocks * 8 == head_dim,
                   "a fused step needs 8-dim blocks of at most 256 centroids");
    const float *cents = static_cast<const float *>(codebook);
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, cents,
                          n_blocks, n_centroids, idx, cap, t_cache, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0, "prepared codebook must be 16-byte aligned");
    SS_REQUIRE(((uintptr_t)centroids % 16) == 0, "centroids must be 16-byte aligned");
    SS_REQUIRE(values_il8, "null values");
    SS_REQUIRE(cap % 8 == 0, "cap must be a multiple of 8 for interleaved values");
    SS_REQUIRE(((uintptr_t)values_il8 % 16) == 0, "values must be 16-byte aligned");
    rc = check_buffer(k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, head_dim);
    if (rc) return rc;
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_cache, n_splits,
                                       kKindMfma);
    DecodeCommon c;
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, cents,
                     n_centroids, idx, cap, t_cache, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    c.centroids = nullptr;
    c.codebook = static_cast<const uint4 *>(codebook);
    c.codebook_mul = reinterpret_cast<const float *>(
        static_cast<const char *>(codebook) + (size_t)cb_tiles(n_blocks, n_centroids) * 2 * kWave * 16);
    if (s.S > 1) {
        // the last split encodes and attends the new tokens before its tiles:
        // it gives up about kStepShareTokens cache tokens to the others, 8 at
        // a time, as far as its own range allows
        const int64_t room = t_cache - (int64_t)(s.S - 1) * s.tiles_per_split * kWave;
        const int64_t want = (kStepShareTokens + (s.S - 1) * 8 - 1) / ((int64_t)(s.S - 1) * 8) * 8;
        const int64_t most = room > 0 ? room / (s.S - 1) / 8 * 8 : 0;
        c.split_pad = (int)(want < most ? want : most);
    }
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    __half *v8 = reinterpret_cast<__half *>(values_il8);
    const float *norms = c.codebook_mul + 4;
    if (head_dim == 128)
        return launch_mfma<128, VIl8Step<128>>(
            c, VIl8Step<128>::Args{v8, k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, centroids,
                                   norms, idx, v8},
            s, st);
    return launch_mfma<64, VIl8Step<64>>(
        c, VIl8Step<64>::Args{v8, k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, centroids, norms,
                              idx, v8},
        s, st);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of ss_decode_attn_il8.  Its split partials and
// per-column counters live in a file-scope device array (one per GPU, held
// until the process ends) instead of a caller workspace.  Host code never
// uses the array's name as an address: the per-device address comes from
// hipGetSymbolAddress at the first call on each device, which also clears
// the counter area with a fill kernel; every completed call leaves it zero.
// ---------------------------------------------------------------------------
constexpr size_t kStaticScratchBytes = 4u << 20;  // 4 MiB per device
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

__global__ void __launch_bounds__(256) zero_words_kernel(uint32_t *p, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// Device address of `scratch` on the current device, looked up (and its
// counter area cleared on `st`) at the first call on that device.
static int static_scratch(void **out, hipStream_t st) {
    static std::mutex mu;
    static void *addr[64] = {nullptr};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    SS_UNSUPPORTED(dev >= 0 && dev < 64, "device ordinal %d beyond 63", dev);
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
        hipLaunchKernelGGL(zero_words_kernel, dim3(64), dim3(256), 0, st,
                           static_cast<uint32_t *>(p), (int64_t)(kCntBytes / 4));
        SS_LAUNCH_CHECK("zero_words_kernel launch");
        addr[dev] = p;
    }
    *out = addr[dev];
    return SS_OK;
}

extern "C" size_t ss_decode_static_scratch_bytes(void) { return kStaticScratchBytes; }

extern "C" int ss_decode_attn_il8_noalloc(const void *q, int q_dtype, int64_t batch,
                                          int n_q_heads, int n_kv_heads, int64_t t_q,
                                          int head_dim, float scale, const int32_t *perm,
                                          const void *codebook, int n_blocks, int n_centroids,
                                          const uint8_t *idx, const void *values_il8,
                                          int v_dtype, int64_t cap, int64_t t_kv, int causal,
                                          int64_t q_offset, void *out, int out_dtype,
                                          int n_splits, void *stream) {
    SS_REQUIRE(batch >= 1 && n_q_heads >= 1 && n_kv_heads >= 1 && t_q >= 1 &&
                   n_q_heads % n_kv_heads == 0,
               "bad head/batch counts");
    SS_UNSUPPORTED(head_dim == 64 || head_dim == 128, "head_dim %d unsupported (64 or 128)",
                   head_dim);
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits,
                                       kKindMfma);
    const size_t need = decode_ws_bytes(s, head_dim);
    if (need > kStaticScratchBytes) {
        set_error("ss_decode_attn_il8_noalloc: this shape needs %zu bytes of split scratch "
                  "(%d splits), the static scratch holds %zu; pass fewer splits or use "
                  "ss_decode_attn_il8 with a workspace",
                  need, s.S, kStaticScratchBytes);
        return SS_ERR_WORKSPACE;
    }
    void *ws = nullptr;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    if (need > 0) {
        const int rc = static_scratch(&ws, st);
        if (rc) return rc;
    }
    return ss_decode_attn_il8(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale,
                              perm, codebook, n_blocks, n_centroids, idx, values_il8, v_dtype,
                              cap, t_kv, causal, q_offset, out, out_dtype, ws,
                              need > 0 ? kStaticScratchBytes : 0, n_splits, stream);
}

static int grouped_il_impl(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                           int n_kv_heads, int64_t t_q, int head_dim, float scale,
                           const int32_t *perm, const void *codebook, int n_blocks,
                           int n_centroids, const uint8_t *idx, const uint32_t *codes_il,
                           const void *scales, const void *zeros, int sz_dtype, int bits,
                           int group_size, int64_t cap, int64_t t_kv, int causal,
                           int64_t q_offset, void *out, int out_dtype, void *workspace,
                           size_t workspace_bytes, int n_splits, const void *k_buf,
                           const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
                           int64_t buf_st, int64_t t_buf, void *stream,
                           const void *k_heavy = nullptr, const int32_t *heavy_dims = nullptr,
                           int n_heavy_dims = 0) {
    const float *cents = static_cast<const float *>(codebook);
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, cents,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(codes_il && scales && zeros, "null codes/scales/zeros");
    SS_UNSUPPORTED(bits == 2 || bits == 4, "interleaved grouped values need bits 2 or 4 (got %d)",
                   bits);
    SS_UNSUPPORTED(group_size == head_dim || 2 * group_size == head_dim,
                   "group_size %d: the fused kernel takes one or two groups per row", group_size);
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(cap % 16 == 0, "cap must be a multiple of 16 for interleaved grouped values");
    SS_REQUIRE(((uintptr_t)codes_il % 16) == 0 && ((uintptr_t)scales % 16) == 0 &&
                   ((uintptr_t)zeros % 16) == 0,
               "codes, scales and zeros must be 16-byte aligned");
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0, "prepared codebook must be 16-byte aligned");
    const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits,
                                       kKindMfma);
    DecodeCommon c;
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, cents,
                     n_centroids, idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    c.centroids = nullptr;
    c.codebook = static_cast<const uint4 *>(codebook);
    c.codebook_mul = reinterpret_cast<const float *>(
        static_cast<const char *>(codebook) + (size_t)cb_tiles(n_blocks, n_centroids) * 2 * kWave * 16);
    rc = check_buffer(k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, t_buf, head_dim);
    if (rc) return rc;
    rc = set_heavy(c, k_heavy, heavy_dims, n_heavy_dims);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const int ng = head_dim / group_size;
#define SS_GIL(DD, BB, NGG, SZT)                                                              \
    {                                                                                         \
        using VF = VGil<DD, BB, NGG, SZT>;                                                    \
        SS_UNSUPPORTED(c.nhd == 0 || VF::kHeavyCapable,                                       \
                       "fp16 heavy key dims with %d-bit values at head_dim %d", BB, DD);       \
        return launch_mfma<DD, VF>(                                                           \
            c,                                                                                \
            typename VF::Args{codes_il, static_cast<const SZT *>(scales),                     \
                              static_cast<const SZT *>(zeros), k_buf, v_buf, buf_dtype,       \
                              buf_sb, buf_sh, buf_st, t_buf > 0 ? t_buf : 0},                 \
            s, st);                                                                           \
    }
#define SS_GIL_SZ(DD, BB, NGG)                     \
    {                                              \
        if (sz_dtype == SS_F16) SS_GIL(DD, BB, NGG, __half) \
        SS_GIL(DD, BB, NGG, float)                 \
    }
#define SS_GIL_NG(DD, BB)                      \
    {                                          \
        if (ng == 2) SS_GIL_SZ(DD, BB, 2)      \
        SS_GIL_SZ(DD, BB, 1)                   \
    }
    if (head_dim == 128) {
        if (bits == 2) SS_GIL_NG(128, 2)
        SS_GIL_NG(128, 4)
    }
    if (bits == 2) SS_GIL_NG(64, 2)
    SS_GIL_NG(64, 4)
#undef SS_GIL_NG
#undef SS_GIL_SZ
#undef SS_GIL
}

extern "C" int ss_decode_attn_grouped_il(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                         int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                         const int32_t *perm, const void *codebook, int n_blocks,
                                         int n_centroids, const uint8_t *idx,
                                         const uint32_t *codes_il, const void *scales,
                                         const void *zeros, int sz_dtype, int bits,
                                         int group_size, int64_t cap, int64_t t_kv, int causal,
                                         int64_t q_offset, void *out, int out_dtype,
                                         void *workspace, size_t workspace_bytes, int n_splits,
                                         void *stream) {
    return grouped_il_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                           codebook, n_blocks, n_centroids, idx, codes_il, scales, zeros, sz_dtype,
                           bits, group_size, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                           workspace_bytes, n_splits, nullptr, nullptr, SS_F16, 0, 0, 0, 0, stream);
}

extern "C" int ss_decode_attn_grouped_il_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint32_t *codes_il, const void *scales,
    const void *zeros, int sz_dtype, int bits, int group_size, int64_t cap, int64_t t_kv,
    const void *k_buf, const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
    int64_t buf_st, int64_t t_buf, const void *k_heavy, const int32_t *heavy_dims,
    int n_heavy_dims, int causal, int64_t q_offset, void *out, int out_dtype, void *workspace,
    size_t workspace_bytes, int n_splits, void *stream) {
    SS_REQUIRE(t_buf >= 0, "negative buffer length");
    return grouped_il_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                           codebook, n_blocks, n_centroids, idx, codes_il, scales, zeros, sz_dtype,
                           bits, group_size, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                           workspace_bytes, n_splits, k_buf, v_buf, buf_dtype, buf_sb, buf_sh,
                           buf_st, t_buf, stream, k_heavy, heavy_dims, n_heavy_dims);
}

// The checks and launch set-up shared by the hybrid-step entry points:
// step sizes, the buffer window and the new tokens, then the common decode
// arguments and the last split's hand-over of cache tokens.
static int hybrid_step_setup(DecodeCommon &c, DecodeShape &s, const void *q, int q_dtype,
                             int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
                             int head_dim, float scale, const int32_t *perm, const void *codebook,
                             const float *centroids, int n_blocks, int n_centroids,
                             const uint8_t *idx, int64_t cap, int64_t t_kv, const void *k_buf,
                             const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh,
                             int64_t buf_st, int64_t n_buf, int64_t n_flush, const void *k_new,
                             const void *v_new, int kv_dtype, int64_t kv_sb, int64_t kv_sh,
                             int64_t kv_st, int64_t n_new, int causal, int64_t q_offset, void *out,
                             int out_dtype, void *workspace, size_t workspace_bytes, int n_splits,
                             int pad_unit) {
    SS_UNSUPPORTED(n_new >= 1 && n_new <= kMaxStepTokens, "a fused step takes 1..%d new tokens",
                   kMaxStepTokens);
    SS_UNSUPPORTED(n_flush >= 0 && n_flush <= kMaxStepTokens,
                   "a fused hybrid step flushes 0..%d tokens (got %lld)", kMaxStepTokens,
                   (long long)n_flush);
    SS_REQUIRE(n_buf >= n_flush, "n_flush %lld exceeds the %lld buffered tokens", (long long)n_flush,
               (long long)n_buf);
    SS_REQUIRE(t_kv >= 1, "a fused hybrid step needs compressed tokens (t_kv %lld)", (long long)t_kv);
    SS_REQUIRE(t_kv + n_flush <= cap, "flushed tokens [%lld, %lld) past cap %lld", (long long)t_kv,
               (long long)(t_kv + n_flush), (long long)cap);
    SS_UNSUPPORTED(kv_dtype == SS_F16 && buf_dtype == SS_F16,
                   "a fused hybrid step takes a float16 buffer and float16 new tokens");
    SS_REQUIRE(k_new && v_new && centroids, "null new keys, values or centroids");
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0, "prepared codebook must be 16-byte aligned");
    const float *cents = static_cast<const float *>(codebook);
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, centroids,
                          n_blocks, n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    // buffer rows 0 .. n_buf + n_new - 1 are read or written
    rc = check_buffer(k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, n_buf + n_new, head_dim);
    if (rc) return rc;
    rc = check_buffer(k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, head_dim);
    if (rc) return rc;
    s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits, kKindMfma);
    rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, cents,
                     n_centroids, idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace,
                     workspace_bytes, head_dim);
    if (rc) return rc;
    c.centroids = nullptr;
    c.codebook = static_cast<const uint4 *>(codebook);
    c.codebook_mul = reinterpret_cast<const float *>(
        static_cast<const char *>(codebook) + (size_t)cb_tiles(n_blocks, n_centroids) * 2 * kWave * 16);
    if (s.S > 1 && n_flush > 0) {
        // the last split encodes and attends the flushed tokens before its
        // tiles: it gives up some cache tokens to the others, in units of
        // pad_unit tokens (a split must start on a code word: 64 for grouped
        // codes, whose 2-bit words hold 16 tokens; 8 for interleaved fp16)
        const int64_t pu = pad_unit;
        const int64_t room = t_kv - (int64_t)(s.S - 1) * s.tiles_per_split * kWave;
        const int64_t want = (kHybridStepShareTokens + (s.S - 1) * pu - 1) / ((int64_t)(s.S - 1) * pu) * pu;
        const int64_t most = room > 0 ? room / (s.S - 1) / pu * pu : 0;
        c.split_pad = (int)(want < most ? want : most);
    }
    return SS_OK;
}

extern "C" int ss_decode_step_grouped_il_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, const float *centroids,
    int n_blocks, int n_centroids, uint8_t *idx, uint32_t *codes_il, void *scales, void *zeros,
    int sz_dtype, int bits, int group_size, int64_t cap, int64_t t_kv, void *k_buf, void *v_buf,
    int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st, int64_t n_buf, int64_t n_flush,
    const void *k_new, const void *v_new, int kv_dtype, int64_t kv_sb, int64_t kv_sh, int64_t kv_st,
    int64_t n_new, int causal, int64_t q_offset, void *out, int out_dtype, void *workspace,
    size_t workspace_bytes, int n_splits, void *stream) {
    SS_REQUIRE(codes_il && scales && zeros, "null codes, scales or zeros");
    SS_UNSUPPORTED(bits == 2 || bits == 4, "a fused hybrid step takes 2- or 4-bit codes (got %d)",
                   bits);
    SS_UNSUPPORTED(group_size == head_dim || 2 * group_size == head_dim,
                   "group_size %d: the fused kernel takes one or two groups per row", group_size);
    SS_REQUIRE(sz_dtype == SS_F32 || sz_dtype == SS_F16, "scale/zero dtype must be f32 or f16");
    SS_REQUIRE(cap % 16 == 0, "cap must be a multiple of 16 for interleaved grouped values");
    SS_REQUIRE(((uintptr_t)codes_il % 16) == 0 && ((uintptr_t)scales % 16) == 0 &&
                   ((uintptr_t)zeros % 16) == 0,
               "codes, scales and zeros must be 16-byte aligned");
    DecodeCommon c;
    DecodeShape s;
    int rc = hybrid_step_setup(c, s, q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale,
                               perm, codebook, centroids, n_blocks, n_centroids, idx, cap, t_kv,
                               k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, n_buf, n_flush,
                               k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, causal, q_offset,
                               out, out_dtype, workspace, workspace_bytes, n_splits, kWave);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const float *norms = c.codebook_mul + 4;
    const int ng = head_dim / group_size;
#define SS_GSTEP(DD, BB, NGG, SZT)                                                              \
    {                                                                                           \
        using VF = VGilStep<DD, BB, NGG, SZT>;                                                  \
        typename VF::Args a{};                                                                  \
        a.codes = codes_il;                                                                     \
        a.scales = static_cast<const SZT *>(scales);                                            \
        a.zeros = static_cast<const SZT *>(zeros);                                              \
        a.kbuf = k_buf;                                                                         \
        a.vbuf = v_buf;                                                                         \
        a.buf_dtype = buf_dtype;                                                                \
        a.buf_sb = buf_sb;                                                                      \
        a.buf_sh = buf_sh;                                                                      \
        a.buf_st = buf_st;                                                                      \
        a.t_buf = n_buf - n_flush + n_new;                                                      \
        a.knew = k_new;                                                                         \
        a.vnew = v_new;                                                                         \
        a.new_sb = kv_sb;                                                                       \
        a.new_sh = kv_sh;                                                                       \
        a.new_st = kv_st;                                                                       \
        a.n_rem = n_buf - n_flush;                                                              \
        a.n_flush = n_flush;                                                                    \
        a.centroids = centroids;                                                                \
        a.cb_norms = norms;                                                                     \
        a.idx_out = idx;                                                                        \
        a.codes_out = codes_il;                                                                 \
        a.scales_out = static_cast<SZT *>(scales);                                              \
        a.zeros_out = static_cast<SZT *>(zeros);                                                \
        a.kput = k_buf;                                                                         \
        a.vput = v_buf;                                                                         \
        return launch_mfma<DD, VF>(c, a, s, st);                                                \
    }
#define SS_GSTEP_SZ(DD, BB, NGG)                             \
    {                                                        \
        if (sz_dtype == SS_F16) SS_GSTEP(DD, BB, NGG, __half) \
        SS_GSTEP(DD, BB, NGG, float)                         \
    }
#define SS_GSTEP_NG(DD, BB)                  \
    {                                        \
        if (ng == 2) SS_GSTEP_SZ(DD, BB, 2)  \
        SS_GSTEP_SZ(DD, BB, 1)               \
    }
    if (head_dim == 128) {
        if (bits == 2) SS_GSTEP_NG(128, 2)
        SS_GSTEP_NG(128, 4)
    }
    if (bits == 2) SS_GSTEP_NG(64, 2)
    SS_GSTEP_NG(64, 4)
#undef SS_GSTEP_NG
#undef SS_GSTEP_SZ
#undef SS_GSTEP
}

extern "C" int ss_decode_step_il8_hybrid(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, const float *centroids,
    int n_blocks, int n_centroids, uint8_t *idx, void *values_il8, int64_t cap, int64_t t_kv,
    void *k_buf, void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st,
    int64_t n_buf, int64_t n_flush, const void *k_new, const void *v_new, int kv_dtype,
    int64_t kv_sb, int64_t kv_sh, int64_t kv_st, int64_t n_new, int causal, int64_t q_offset,
    void *out, int out_dtype, void *workspace, size_t workspace_bytes, int n_splits, void *stream) {
    SS_REQUIRE(values_il8, "null values");
    SS_REQUIRE(cap % 8 == 0, "cap must be a multiple of 8 for interleaved values");
    SS_REQUIRE(((uintptr_t)values_il8 % 16) == 0, "values must be 16-byte aligned");
    DecodeCommon c;
    DecodeShape s;
    int rc = hybrid_step_setup(c, s, q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale,
                               perm, codebook, centroids, n_blocks, n_centroids, idx, cap, t_kv,
                               k_buf, v_buf, buf_dtype, buf_sb, buf_sh, buf_st, n_buf, n_flush,
                               k_new, v_new, kv_dtype, kv_sb, kv_sh, kv_st, n_new, causal, q_offset,
                               out, out_dtype, workspace, workspace_bytes, n_splits, 8);
    if (rc) return rc;
    hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    const float *norms = c.codebook_mul + 4;
    __half *v8 = static_cast<__half *>(values_il8);
    auto run = [&](auto dtag) {
        constexpr int DD = decltype(dtag)::value;
        using VF = VIl8HybStep<DD>;
        typename VF::Args a{};
        a.v8 = v8;
        a.kbuf = k_buf;
        a.vbuf = v_buf;
        a.buf_dtype = buf_dtype;
        a.buf_sb = buf_sb;
        a.buf_sh = buf_sh;
        a.buf_st = buf_st;
        a.t_buf = n_buf - n_flush + n_new;
        a.knew = k_new;
        a.vnew = v_new;
        a.new_sb = kv_sb;
        a.new_sh = kv_sh;
        a.new_st = kv_st;
        a.n_rem = n_buf - n_flush;
        a.n_flush = n_flush;
        a.centroids = centroids;
        a.cb_norms = norms;
        a.idx_out = idx;
        a.v8_out = v8;
        a.kput = k_buf;
        a.vput = v_buf;
        return launch_mfma<DD, VF>(c, a, s, st);
    };
    if (head_dim == 128) return run(std::integral_constant<int, 128>{});
    return run(std::integral_constant<int, 64>{});
}

extern "C" int ss_decode_attn_turboquant_il(
    const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads, int64_t t_q,
    int head_dim, float scale, const int32_t *perm, const void *codebook, int n_blocks,
    int n_centroids, const uint8_t *idx, const uint32_t *codes_il, const float *norms,
    const float *levels, const float *rotation, int64_t cap, int64_t t_kv, const void *k_buf,
    const void *v_buf, int buf_dtype, int64_t buf_sb, int64_t buf_sh, int64_t buf_st, int64_t t_buf,
    const void *k_heavy, const int32_t *heavy_dims, int n_heavy_dims, int causal, int64_t q_offset,
    void *out, int out_dtype, void *workspace, size_t workspace_bytes, int n_splits, void *stream) {
    const float *cents = static_cast<const float *>(codebook);
    int rc = check_common(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, cents, n_blocks,
                          n_centroids, idx, cap, t_kv, out, out_dtype);
    if (rc) return rc;
    SS_REQUIRE(codes_il && norms && levels && rotation, "null codes/norms/levels/rotation");
    SS_REQUIRE(cap % 16 == 0, "cap must be a multiple of 16 for interleaved 2-bit codes");
    SS_REQUIRE(((uintptr_t)codes_il % 16) == 0 && ((uintptr_t)norms % 16) == 0,
               "codes and norms must be 16-byte aligned");
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0, "prepared codebook must be 16-byte aligned");
    // the levels must be affine in the two code bits (a symmetric table)
    const float lmax = fmaxf(fmaxf(fabsf(levels[0]), fabsf(levels[3])), 1e-30f);
    SS_UNSUPPORTED(fabsf(levels[3] - (levels[2] + levels[1] - levels[0])) <= 1e-6f * lmax,
                   "2-bit levels are not affine in the code bits (L3 != L2 + L1 - L0)");
    typename VTq<128>::Args va128{codes_il, norms, levels[0], levels[1] - levels[0],
                                  levels[2] - 2.f * levels[1] + levels[0]};
    // fused: the kernel writes out itself, rotated (one split, or its
    // in-kernel merge); else split partials that transformed_decode merges
    // with the buffer's partial and rotates
    auto launch_tq = [&](const DecodeCommon &c0, const DecodeShape &s, hipStream_t st,
                         bool fused) -> int {
        DecodeCommon c = c0;
        c.centroids = nullptr;
        c.codebook = static_cast<const uint4 *>(codebook);
        c.codebook_mul = reinterpret_cast<const float *>(
            static_cast<const char *>(codebook) + (size_t)cb_tiles(n_blocks, n_centroids) * 2 * kWave * 16);
        if (fused)
            c.rot = rotation;
        else
            c.fused_merge = 0;
        const int hrc = set_heavy(c, k_heavy, heavy_dims, n_heavy_dims);
        if (hrc) return hrc;
        auto go = [&](auto dd, auto vf) -> int {
            constexpr int DD = decltype(dd)::value;
            using VF = typename decltype(vf)::type;
            constexpr int NC = VF::kComputeWaves;
            using K = WsCfg<DD, NC, VF>;
            auto kern = decode_attn_mfma_kernel<DD, NC, VF>;
            const int src = mfma_kernel_setup<DD, VF>();
            if (src) return src;
            const typename VF::Args va{va128.codes, va128.norms, va128.l0, va128.l1, va128.l2};
            hipLaunchKernelGGL(kern, dim3(s.S, s.n_cols), dim3(K::kWaves * kWave), K::kLds, st, c, va);
            SS_LAUNCH_CHECK("decode_attn_mfma_kernel (turboquant) launch");
            return SS_OK;
        };
        using I128 = std::integral_constant<int, 128>;
        using I64 = std::integral_constant<int, 64>;
        if (c.nhd > 0)
            return head_dim == 128 ? go(I128{}, TypeTag<WithHeavy<VTq<128>>>{})
                                   : go(I64{}, TypeTag<WithHeavy<VTq<64>>>{});
        return head_dim == 128 ? go(I128{}, TypeTag<VTq<128>>{})
                               : go(I64{}, TypeTag<VTq<64>>{});
    };
    if (t_buf == 0) {
        // no buffered tokens: one launch, rotation applied by the kernel
        const DecodeShape s = decode_shape(batch, n_q_heads, n_kv_heads, t_q, t_kv, n_splits, kKindMfma);
        DecodeCommon c;
        rc = fill_common(c, s, q, q_dtype, n_q_heads, n_kv_heads, t_q, scale, perm, cents, n_centroids,
                         idx, cap, t_kv, causal, q_offset, out, out_dtype, workspace, workspace_bytes,
                         head_dim);
        if (rc) return rc;
        SS_REQUIRE(((uintptr_t)rotation % 4) == 0, "misaligned rotation matrix");
        if (s.S == 1 || c.fused_merge)
            return launch_tq(c, s, reinterpret_cast<hipStream_t>(stream), true);
    }
    auto main = [&](const DecodeCommon &c0, const DecodeShape &s, hipStream_t st) -> int {
        return launch_tq(c0, s, st, false);
    };
    return transformed_decode(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm, cents,
                              n_centroids, idx, cap, t_kv, rotation, k_buf, v_buf, buf_dtype, buf_sb, buf_sh,
                              buf_st, t_buf, causal, q_offset, out, out_dtype, workspace, workspace_bytes,
                              n_splits, stream, main, kKindMfma);
}
