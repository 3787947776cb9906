// Causal prefill attention over block-VQ keys and 8-token interleaved fp16
// values: the prompt's query rows (T_q of them per query head) against the
// cache that holds them, the shape of the reference's fused causal kernels
// (kernels.py:303-378) at T_q > 1, reorganised for the matrix cores.
//
// A decode kernel builds one query x centroid LUT per 4 query rows and
// gathers scores from it; for a prompt that means one LUT and one pass over
// the cache prefix per 4 rows.  Here the keys are reconstructed instead: the
// prepared split-fp16 codebook (hi + lo * 2^-11 of C * 2^-e, the operand of
// the decode kernels' LUT build) is copied row-major into LDS once per
// workgroup, and the scores of 16 tokens x 16 query rows are
//   S^T[token][row] = sum_k Khat[token][k] * Q'[row][k]
// on v_mfma_f32_16x16x32_f16: A = the tokens' codebook rows (lane l holds
// block 4*ks + l/16 of token l%16: one 16-byte LDS read each for hi and lo),
// B = the query rows (round_to(q_dtype, q * scale), codec-permuted, as
// registers for the whole kernel; fp16 hi and lo parts unless the query is
// fp16).  The accumulator of S^T gives lane l the scores of row l%16 for
// tokens 4*(l/16) .. +3 of each 16-token sub-tile; two sub-tiles' entries
// side by side are an A operand of
//   O[row][dim] += sum_t P[row][t] * V[t][dim]
// on v_mfma_f32_16x16x32_f16 (the token order inside a product's K slots
// is free as long as A and B agree), so the probabilities never leave
// registers (hi and lo fp16 parts of p * 2^11, two products); B = the same 8
// tokens of one dim, two 8-byte loads of the interleaved value layout.
//
// A workgroup of kPfWaves waves takes 16 * kPfWaves query rows of one KV
// group: (rows / rep) consecutive positions of its rep query heads, the
// heads sharing every key and value read.  Each wave owns 16 rows outright
// (its own online softmax and accumulators), so there is no split, merge or
// cross-wave combine.  Causal rows stop at q_offset + position.
//
// fp16 and bf16 queries take prefill32_il8_kernel instead: waves of 32 rows on
// v_mfma_f32_32x32x16_f16 (S^T of 32 tokens x 32 rows: lane l holds token
// l%32's block 2ks + l/32 as A, row l%32's dims 16ks + 8(l/32) .. as B) and
// v_mfma_f32_32x32x16_f16 for P.V too (the S^T accumulator entries 8k2 ..
// 8k2+7 of lane l are row l%32's tokens 16k2 + 4(l/32) + 0..3 and
// 16k2 + 8 + 4(l/32) + 0..3, the A operand of step k2; the legacy
// 32x32x8 and 16x16x16 shapes issue at half the fp16 rate on gfx950), so
// every key gather and value load serves 32 rows.  There the key's hi and
// lo parts accumulate into one S (the lo rows taken back to the hi units
// in LDS) and P enters P.V as one fp16 operand (p * 2^11 rounded: each
// weight within 2^-12 of itself), one product per k-step.  fp32 queries
// need a second (lo) query operand, which leaves no registers for 32 rows.
//
// The grid is (batch x KV heads, position groups) with the position groups
// in reverse order along y: workgroups are dispatched x fastest, so the
// heaviest causal ranges of every head go first.
#include "ss_common.hpp"

#include <type_traits>

namespace ss {

namespace {

typedef _Float16 pf_f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 pf_f16x8 __attribute__((ext_vector_type(8)));
typedef float pf_f32x4 __attribute__((ext_vector_type(4)));
typedef float pf_f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 pf_f16x2 __attribute__((ext_vector_type(2)));
typedef float pf_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPfWaves = 8;
constexpr int kPfRows = 16 * kPfWaves;   // query rows of a workgroup (16 per wave)
constexpr int kPfRows32 = 32 * kPfWaves; // the same with 32 rows per wave (fp16 queries)
constexpr int kPfD = 128;
constexpr int kPfNB = 16;
constexpr int kPfRows16 = kPfNB * 256;   // codebook rows (block, centroid), 16 bytes each
constexpr int kPfLdsBytes = 2 * kPfRows16 * 16;  // hi rows, then lo rows: 128 KB
constexpr float kPfSplit = 2048.f;       // lo parts carry 2^11
// A row keeps its running maximum while a tile's scores stay within kPfLag
// log2 units above it (no rescale of its accumulators); its probabilities,
// staged as fp16 hi/lo of p * 2^kPfPExp, then reach 2^(kPfPExp + kPfLag),
// below the fp16 maximum.
constexpr float kPfLag = 4.f;
constexpr float kPfPExp = 11.f;

struct PrefillArgs {
    const void *q;
    int q_dtype;
    int n_q_heads, n_kv_heads, rep;
    int64_t t_q;
    float scale;
    const int32_t *perm;
    const uint4 *codebook;   // prepared split-fp16 tiles (ss_codebook_f16x2)
    const float *cb_mul;     // their power-of-two multiplier
    int nct;                 // centroid tiles of 16
    const uint8_t *idx;      // [B][Hkv][cap][16]
    const __half *v8;        // [B][Hkv][cap_v/8][128][8]
    int64_t cap, cap_v, t_kv;
    // keys from position t_raw0 on (a hybrid cache's buffered tokens) are
    // given whole instead of as indices: kraw [B][Hkv][n_raw][2][128] fp16,
    // per token its codec-basis key times 2^-s (hi) and the remainder (lo),
    // kfac [B][Hkv][n_raw] = 2^s; t_raw0 = t_kv when there are none
    const __half *kraw;
    const float *kfac;
    int64_t t_raw0, n_raw;
    int causal;
    int64_t q_offset;
    void *out;
    int out_dtype;
    int npos;                // positions per workgroup = rows per workgroup / rep
    int n_pg;                // position groups
};

// x of lane `src` (0..63) of this wave
__device__ __forceinline__ float lane_read(float x, int src) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src << 2, __float_as_int(x)));
}

__device__ __forceinline__ float xor_max(float x, int m) {
    return fmaxf(x, __shfl_xor(x, m));
}

}  // namespace

__global__ void __launch_bounds__(kPfWaves * kWave) prefill16_il8_kernel(PrefillArgs a) {
    constexpr int TH = kPfWaves * kWave;
    extern __shared__ __align__(16) float4 pf_smem[];
    char *lds = reinterpret_cast<char *>(pf_smem);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    // the longest causal ranges first: position groups in reverse order
    // along y, the (batch, KV head) columns along x, so that workgroups are
    // dispatched heaviest position group first across every head
    const int pg = a.n_pg - 1 - (int)blockIdx.y;
    const int64_t bh = blockIdx.x;
    const int64_t bb = bh / a.n_kv_heads;
    const int kvh = (int)(bh - bb * a.n_kv_heads);

    // 1. the prepared codebook, row-major: the hi part of row (block,
    //    centroid) at (block * 256 + centroid) * 16 bytes, its lo part 64 KB
    //    further (16-byte rows spread random gathers over 16 bank groups).
    //    Tile t = (bg, ct) holds 64 lanes' rows: block bg*4 + l/16, centroid
    //    ct*16 + l%16.
    uint4 *lds4 = reinterpret_cast<uint4 *>(lds);
    for (int i = tid; i < 4 * a.nct * kWave; i += TH) {
        const int t = i >> 6, l = i & 63, bg = t / a.nct, ct = t - bg * a.nct;
        const int row = (bg * 4 + (l >> 4)) * 256 + ct * 16 + (l & 15);
        lds4[row] = a.codebook[(int64_t)t * 2 * kWave + l];
        lds4[kPfRows16 + row] = a.codebook[(int64_t)t * 2 * kWave + kWave + l];
    }

    // 2. this lane's query row (the S^T column l%16 of wave wv): B operands
    //    of the 4 k-steps, dims 32*ks + 8*g .. +7, codec-permuted
    const int r = wv * 16 + l16;
    const int p = r / a.rep, h = r - p * a.rep;
    const int64_t pos = (int64_t)pg * a.npos + p;
    const bool rok = pos < a.t_q;
    const int64_t qoff = ((bb * a.n_q_heads + (int64_t)kvh * a.rep + h) * a.t_q + (rok ? pos : 0)) *
                         kPfD;
    // the row enters scaled by a power of two 2^-s that brings its largest
    // element into [2^14, 2^15), so the fp16 hi part never overflows (the
    // scores are multiplied back by 2^s in the exponent below)
    auto q_at = [&](int j) {
        const int src = a.perm ? min(max(a.perm[j], 0), kPfD - 1) : j;
        return rok ? round_to(a.q_dtype, load_as_f32(a.q, a.q_dtype, qoff + src) * a.scale) : 0.f;
    };
    float qmax = 0.f;
    for (int j = 8 * g; j < kPfD; j += 32)
#pragma unroll
        for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(q_at(j + e)));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 16));  // lanes l16 + 16 g hold the row's quarters
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));
    const int qshift = row_exp_shift(qmax);
    const float qinv = exp2i(-qshift);
    pf_f16x8 qh[4], ql[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = q_at(32 * ks + 8 * g + e) * qinv;
            const _Float16 hx = (_Float16)x;
            qh[ks][e] = hx;
            ql[ks][e] = (_Float16)((x - (float)hx) * kPfSplit);
        }
    const bool qsplit = a.q_dtype != SS_F16;
    __syncthreads();
    // a wave whose rows all lie past the prompt has nothing to do (no
    // barrier follows)
    const int64_t wave_pos0 = (int64_t)pg * a.npos + (wv * 16) / a.rep;
    if (wave_pos0 >= a.t_q) return;

    // scores stay in the prepared codebook's units (hi + lo * 2^-11) and the
    // row's query scale; mul takes them to log2 units inside the exponent
    const float mul = *a.cb_mul * kLog2e * exp2i(qshift);
    // keys this workgroup reads: causal rows stop at q_offset + position
    const int64_t pos_last = min((int64_t)(pg + 1) * a.npos, a.t_q) - 1;
    const int64_t t_end = a.causal ? min(a.t_kv, a.q_offset + pos_last + 1) : a.t_kv;
    // token indices below are 32-bit (cap < 2^24 checked on the host)
    const int t_end32 = (int)t_end;
    // this lane's row limit; rows past the prompt are never stored, so they
    // need no mask
    const int lim32 = (!rok || !a.causal) ? 0x7fffffff : (int)(a.q_offset + pos);
    // the wave's smallest limit: tiles entirely below it need no mask
    const int lim_min32 = a.causal ? (int)(a.q_offset + wave_pos0) : 0x7fffffff;
    const int n_tiles = t_end32 > 0 ? (t_end32 + kWave - 1) / kWave : 0;
    const int t_last = max(t_end32 - 1, 0);
    const uint8_t *idx_head = a.idx + bh * a.cap * kPfNB;
    const char *v_head = reinterpret_cast<const char *>(a.v8 + bh * a.cap_v * kPfD);

    float m = -1e30f, lsum = 0.f;  // row l16 (lsum: this lane's share)
    pf_f32x4 acc[8];
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) acc[nt] = pf_f32x4{0.f, 0.f, 0.f, 0.f};

    auto load_idx = [&](uint4 (&ir)[4], int tile) {
        const int t0 = tile * kWave;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            ir[j] = *reinterpret_cast<const uint4 *>(
                idx_head + (uint32_t)min(t0 + 16 * j + l16, t_last) * kPfNB);
    };
    uint4 ir_a[4], ir_b[4];
    if (n_tiles > 0) load_idx(ir_a, 0);

    auto do_tile = [&](const uint4 (&ir_cur)[4], uint4 (&ir_nxt)[4], int tile) {
        const int t0 = tile * kWave;
        // the tile's value operands (4 tokens of one dim, 8 bytes), issued
        // first so they land while the scores are computed; 8-token blocks
        // past the last key clamp to its block (their weights are zero)
        uint2 vop[4][8];
        const int blk_last = t_last >> 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t blk = (uint32_t)min((t0 + 16 * j + 4 * g) >> 3, blk_last);
            const uint32_t off = ((blk * kPfD + l16) * 8 + ((4 * g) & 7)) * 2;
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
                vop[j][nt] = *reinterpret_cast<const uint2 *>(v_head + off + nt * 256);
        }
        load_idx(ir_nxt, min(tile + 1, n_tiles - 1));
        // scores S^T of 4 sub-tiles of 16 tokens, log2 units; a tile below
        // every row's limit and the last key is not masked (wave-uniform)
        const bool full = t0 + kWave - 1 < t_end32 && t0 + kWave - 1 <= lim_min32;
        const int rem_end = t_end32 - t0 - 4 * g, rem_lim = lim32 == 0x7fffffff ? 0x7fffffff
                                                                             : lim32 - t0 - 4 * g;
        float sv[4][4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            pf_f32x4 sh = pf_f32x4{0.f, 0.f, 0.f, 0.f}, sl = sh;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                const uint32_t w = ks == 0 ? ir_cur[j].x : ks == 1 ? ir_cur[j].y
                                 : ks == 2 ? ir_cur[j].z : ir_cur[j].w;
                const uint32_t c = __builtin_amdgcn_ubfe(w, 8 * g, 8);
                const char *row = lds + ((4 * ks + g) * 256 + c) * 16;
                const pf_f16x8 ah = *reinterpret_cast<const pf_f16x8 *>(row);
                const pf_f16x8 al = *reinterpret_cast<const pf_f16x8 *>(row + kPfRows16 * 16);
                sh = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qh[ks], sh, 0, 0, 0);
                sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, qh[ks], sl, 0, 0, 0);
                if (qsplit) sl = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, ql[ks], sl, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sv[j][i] = fmaf(sl[i], 1.f / kPfSplit, sh[i]);
            if (!full) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int k = 16 * j + i;
                    sv[j][i] = (k < rem_end && k <= rem_lim) ? sv[j][i] : -INFINITY;
                }
            }
        }
        // online softmax of row l16 over the tile's 64 tokens (16 here, the
        // rest in lanes l16 + 16, + 32, + 48)
        float mx = sv[0][0];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) mx = fmaxf(mx, sv[j][i]);
        mx = xor_max(mx, 16);
        mx = xor_max(mx, 32);
        const float mn = (mx - m) * mul > kPfLag ? fmaxf(m, mx) : m;  // raw units (mul > 0)
        const float corr = fast_exp2((m - mn) * mul);
        m = mn;
        // x = p * 2^11 = exp2(s * mul - (mn * mul - 11)), split into fp16 hi
        // and lo; l sums x and is scaled back at the end
        float ps = 0.f;
        const float off = fmaf(mn, mul, -kPfPExp);
        pf_f16x4 phi[4], plo[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float x = fast_exp2(fmaf(sv[j][i], mul, -off));
                ps += x;
                const _Float16 hx = (_Float16)x;
                phi[j][i] = hx;
                plo[j][i] = (_Float16)__builtin_fmaf((float)hx, -1.f, x);
            }
        lsum = fmaf(lsum, corr, ps);
        // accumulator rows 4g + i take the correction of their own rows
        if (__builtin_amdgcn_ballot_w64(corr != 1.f) != 0) {
            pf_f32x4 c4;
#pragma unroll
            for (int i = 0; i < 4; ++i) c4[i] = __shfl(corr, 4 * g + i);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) acc[nt] *= c4;
        }
        if (t0 + kWave > t_end32) {  // the last tile (wave-uniform)
            // zero the values of tokens past the last key (their weights are
            // zero, the stale halves need not be finite)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int n_ok = max(min(rem_end - 16 * j, 4), 0);
                const uint32_t mx_ = n_ok >= 2 ? 0xffffffffu : n_ok == 1 ? 0x0000ffffu : 0u;
                const uint32_t my_ = n_ok >= 4 ? 0xffffffffu : n_ok == 3 ? 0x0000ffffu : 0u;
#pragma unroll
                for (int nt = 0; nt < 8; ++nt) {
                    vop[j][nt].x &= mx_;
                    vop[j][nt].y &= my_;
                }
            }
        }
        // P.V on v_mfma_f32_16x16x32_f16: step j2 takes the 32 tokens of
        // sub-tiles 2j2 and 2j2+1, the lane's eight being its four of each;
        // its B slice holds the same eight tokens' values (slot for slot)
#pragma unroll
        for (int j2 = 0; j2 < 2; ++j2) {
            const pf_f16x8 ah = __builtin_shufflevector(phi[2 * j2], phi[2 * j2 + 1], 0, 1, 2, 3, 4, 5, 6, 7);
            const pf_f16x8 al = __builtin_shufflevector(plo[2 * j2], plo[2 * j2 + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < 8; ++nt) {
                const pf_f16x8 b = __builtin_bit_cast(
                    pf_f16x8, make_uint4(vop[2 * j2][nt].x, vop[2 * j2][nt].y, vop[2 * j2 + 1][nt].x,
                                         vop[2 * j2 + 1][nt].y));
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, acc[nt], 0, 0, 0);
                acc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, b, acc[nt], 0, 0, 0);
            }
        }
    };
    for (int tile = 0; tile < n_tiles; tile += 2) {
        do_tile(ir_a, ir_b, tile);
        if (tile + 1 >= n_tiles) break;
        do_tile(ir_b, ir_a, tile + 1);
    }

    // 3. rows 4g + i of the accumulators: their l (the row's four lane
    //    shares summed), then the output
    float L = lsum + __shfl_xor(lsum, 16);
    L += __shfl_xor(L, 32);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float Li = __shfl(L, 4 * g + i);
        const int rr = wv * 16 + 4 * g + i;
        const int pp = rr / a.rep, hh = rr - pp * a.rep;
        const int64_t opos = (int64_t)pg * a.npos + pp;
        if (opos < a.t_q) {
            const int64_t off =
                ((bb * a.n_q_heads + (int64_t)kvh * a.rep + hh) * a.t_q + opos) * kPfD;
            const float inv = Li > 0.f ? 1.f / Li : 0.f;  // acc and l both carry 2^11
#pragma unroll
            for (int nt = 0; nt < 8; ++nt)
                store_from_f32(a.out, a.out_dtype, off + 16 * nt + l16, acc[nt][i] * inv);
        }
    }
}

__global__ void __launch_bounds__(kPfWaves * kWave) prefill32_il8_kernel(PrefillArgs a) {
    constexpr int TH = kPfWaves * kWave;
    extern __shared__ __align__(16) float4 pf_smem[];
    char *lds = reinterpret_cast<char *>(pf_smem);
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hb = lane >> 5, l32 = lane & 31;
    // the longest causal ranges first: position groups in reverse order
    const int pg = a.n_pg - 1 - (int)blockIdx.y;
    const int64_t bh = blockIdx.x;
    const int64_t bb = bh / a.n_kv_heads;
    const int kvh = (int)(bh - bb * a.n_kv_heads);

    // 1. the prepared codebook, row-major: the hi part of row (block,
    //    centroid) at (block * 256 + centroid) * 16 bytes, its lo part 64 KB
    //    further, taken back to the hi part's units (lo * 2^-11, exact but
    //    for lo parts below fp16's normal range, which are under 2^-38 of
    //    the largest hi part) so both products accumulate into one S.
    //    Tile t = (bg, ct) holds 64 lanes' rows: block bg*4 + l/16,
    //    centroid ct*16 + l%16.
    uint4 *lds4 = reinterpret_cast<uint4 *>(lds);
    for (int i = tid; i < 4 * a.nct * kWave; i += TH) {
        const int t = i >> 6, l = i & 63, bg = t / a.nct, ct = t - bg * a.nct;
        const int row = (bg * 4 + (l >> 4)) * 256 + ct * 16 + (l & 15);
        lds4[row] = a.codebook[(int64_t)t * 2 * kWave + l];
        const pf_f16x8 lo = __builtin_bit_cast(pf_f16x8, a.codebook[(int64_t)t * 2 * kWave + kWave + l]) *
                            (_Float16)(1.f / kPfSplit);
        lds4[kPfRows16 + row] = __builtin_bit_cast(uint4, lo);
    }

    // 2. this lane's query row (the S^T column l%32 of wave wv): B operands
    //    of the 8 k-steps, dims 16*ks + 8*hb .. +7, codec-permuted
    const int r = wv * 32 + l32;
    const int p = r / a.rep, h = r - p * a.rep;
    const int64_t pos = (int64_t)pg * a.npos + p;
    const bool rok = pos < a.t_q;
    const int64_t qoff = ((bb * a.n_q_heads + (int64_t)kvh * a.rep + h) * a.t_q + (rok ? pos : 0)) *
                         kPfD;
    // the row enters scaled by a power of two 2^-s that brings its largest
    // element into [2^14, 2^15): fp16 and bf16 elements are then exact in
    // fp16 (down to 2^-29 of the largest), whatever the row's magnitude, and
    // the scores are multiplied back by 2^s in the exponent below
    auto q_at = [&](int j) {
        const int src = a.perm ? min(max(a.perm[j], 0), kPfD - 1) : j;
        return rok ? round_to(a.q_dtype, load_as_f32(a.q, a.q_dtype, qoff + src) * a.scale) : 0.f;
    };
    float qmax = 0.f;
    for (int j = 8 * hb; j < kPfD; j += 16)
#pragma unroll
        for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(q_at(j + e)));
    qmax = fmaxf(qmax, __shfl_xor(qmax, 32));  // lanes l and l ^ 32 hold the row's two halves
    const int qshift = row_exp_shift(qmax);
    const float qinv = exp2i(-qshift);
    pf_f16x8 qh[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks)
#pragma unroll
        for (int e = 0; e < 8; ++e) qh[ks][e] = (_Float16)(q_at(16 * ks + 8 * hb + e) * qinv);
    __syncthreads();
    // a wave whose rows all lie past the prompt has nothing to do (no
    // barrier follows)
    const int64_t wave_pos0 = (int64_t)pg * a.npos + (wv * 32) / a.rep;
    if (wave_pos0 >= a.t_q) return;

    // scores stay in the prepared codebook's units (hi + lo * 2^-11) and the
    // row's query scale; mul takes them to log2 units inside the exponent
    const float mul = *a.cb_mul * kLog2e * exp2i(qshift);
    // keys this workgroup reads: causal rows stop at q_offset + position
    const int64_t pos_last = min((int64_t)(pg + 1) * a.npos, a.t_q) - 1;
    const int64_t t_end = a.causal ? min(a.t_kv, a.q_offset + pos_last + 1) : a.t_kv;
    // token indices below are 32-bit (cap < 2^24 checked on the host)
    const int t_end32 = (int)t_end;
    // this lane's row limit; rows past the prompt are never stored, so they
    // need no mask
    const int lim32 = (!rok || !a.causal) ? 0x7fffffff : (int)(a.q_offset + pos);
    // the wave's smallest limit: sub-tiles entirely below it need no mask
    const int lim_min32 = a.causal ? (int)(a.q_offset + wave_pos0) : 0x7fffffff;
    const int n_sub = t_end32 > 0 ? (t_end32 + 31) / 32 : 0;
    const int t_last = max(t_end32 - 1, 0);
    const uint8_t *idx_head = a.idx + bh * a.cap * kPfNB;
    const char *v_head = reinterpret_cast<const char *>(a.v8 + bh * a.cap_v * kPfD);
    // whole keys from position t_raw0 on (none without kraw: no sub-tile
    // reaches INT_MAX); index rows only below it
    const int t_raw0 = a.kraw ? (int)a.t_raw0 : INT_MAX;
    const int idx_last = max(min(t_last, t_raw0 - 1), 0);
    const int n_raw32 = (int)max(a.n_raw, (int64_t)1);
    const __half *kraw_head = a.kraw ? a.kraw + bh * a.n_raw * 2 * kPfD : nullptr;
    const float *kfac_head = a.kfac ? a.kfac + bh * a.n_raw : nullptr;
    const float inv_cb_mul = 1.f / *a.cb_mul;  // a power of two

    float m = -1e30f, lsum = 0.f;  // row l32 (lsum: this lane's half of its tokens)
    pf_f32x16 acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[nt][i] = 0.f;

    // the index row of token t0 + l32 (both lane halves read the same row)
    auto load_idx = [&](uint4 &ir, int sub) {
        ir = *reinterpret_cast<const uint4 *>(idx_head + (uint32_t)min(32 * sub + l32, idx_last) * kPfNB);
    };
    uint4 ir_a, ir_b;
    if (n_sub > 0) load_idx(ir_a, 0);

    // raw_c: std::true_type for the sub-tiles that may reach the whole keys
    // (from t_raw0 on), which get the per-lane key source; the others
    // compile without it
    auto do_sub = [&](auto raw_c, const uint4 &ir_cur, uint4 &ir_nxt, int sub)
                      __attribute__((always_inline)) {
        constexpr bool kRaw = decltype(raw_c)::value;
        const int t0 = 32 * sub;
        // the sub-tile's value operands (4 tokens of one dim, 8 bytes) for the
        // 4 steps of 8 tokens and 4 n-tiles of 32 dims, issued first so they
        // land while the scores are computed; 8-token blocks past the last
        // key clamp to its block (their weights are zero)
        uint2 vop[4][4];
        const int blk_last = t_last >> 3;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            const uint32_t blk = (uint32_t)min((t0 + 8 * kk) >> 3, blk_last);
            const uint32_t off = ((blk * kPfD + l32) * 8 + 4 * hb) * 2;
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                vop[kk][nt] = *reinterpret_cast<const uint2 *>(v_head + off + nt * 512);
        }
        load_idx(ir_nxt, min(sub + 1, n_sub - 1));
        // scores S^T[token][row] of 32 tokens x 32 rows: lane l holds row
        // l%32 and tokens 8*(i/4) + 4*hb + i%4 (i = 0..15); the hi and lo
        // parts of the keys accumulate into the same S
        pf_f32x16 sv;
#pragma unroll
        for (int i = 0; i < 16; ++i) sv[i] = 0.f;
        // a sub-tile reaching the whole keys (wave-uniform): lanes whose
        // token is past t_raw0 take its key rows from kraw
        const bool raw_tile = kRaw && t0 + 31 >= t_raw0;
        if (!raw_tile) {
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int blk = 2 * ks + hb;
                const uint32_t w = (blk >> 2) == 0 ? ir_cur.x : (blk >> 2) == 1 ? ir_cur.y
                                 : (blk >> 2) == 2 ? ir_cur.z : ir_cur.w;
                const uint32_t c = __builtin_amdgcn_ubfe(w, 8 * (blk & 3), 8);
                const char *row = lds + (blk * 256 + c) * 16;
                const pf_f16x8 ah = *reinterpret_cast<const pf_f16x8 *>(row);
                const pf_f16x8 al = *reinterpret_cast<const pf_f16x8 *>(row + kPfRows16 * 16);
                sv = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[ks], sv, 0, 0, 0);
                sv = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[ks], sv, 0, 0, 0);
            }
        } else {
            const int tk = t0 + l32;
            const bool mine_raw = tk >= t_raw0;
            const __half *kr = kraw_head + (uint32_t)min(max(tk - t_raw0, 0), n_raw32 - 1) * 2 * kPfD;
#pragma unroll
            for (int ks = 0; ks < 8; ++ks) {
                const int blk = 2 * ks + hb;
                pf_f16x8 ah, al;
                if (mine_raw) {
                    ah = *reinterpret_cast<const pf_f16x8 *>(kr + blk * 8);
                    al = *reinterpret_cast<const pf_f16x8 *>(kr + kPfD + blk * 8);
                } else {
                    const uint32_t w = (blk >> 2) == 0 ? ir_cur.x : (blk >> 2) == 1 ? ir_cur.y
                                     : (blk >> 2) == 2 ? ir_cur.z : ir_cur.w;
                    const uint32_t c = __builtin_amdgcn_ubfe(w, 8 * (blk & 3), 8);
                    const char *row = lds + (blk * 256 + c) * 16;
                    ah = *reinterpret_cast<const pf_f16x8 *>(row);
                    al = *reinterpret_cast<const pf_f16x8 *>(row + kPfRows16 * 16);
                }
                sv = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qh[ks], sv, 0, 0, 0);
                sv = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qh[ks], sv, 0, 0, 0);
            }
        }
        if (raw_tile) {
            // whole keys' scores into the codebook's units: times their own
            // 2^s and the codebook's power of two
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tk = t0 + 8 * (i >> 2) + 4 * hb + (i & 3);
                if (tk >= t_raw0)
                    sv[i] *= kfac_head[min(tk - t_raw0, n_raw32 - 1)] * inv_cb_mul;
            }
        }
        // a sub-tile below every row's limit and the last key is not masked
        // (wave-uniform)
        const bool full = t0 + 31 < t_end32 && t0 + 31 <= lim_min32;
        if (!full) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int tk = t0 + 8 * (i >> 2) + 4 * hb + (i & 3);
                sv[i] = (tk < t_end32 && tk <= lim32) ? sv[i] : -INFINITY;
            }
        }
        // online softmax of row l32 over the sub-tile's 32 tokens (16 here,
        // 16 in lane l ^ 32)
        float mx = sv[0];
#pragma unroll
        for (int i = 1; i < 16; ++i) mx = fmaxf(mx, sv[i]);
        mx = fmaxf(mx, lane_read(mx, lane ^ 32));
        const float mn = (mx - m) * mul > kPfLag ? fmaxf(m, mx) : m;  // raw units (mul > 0)
        const float corr = fast_exp2((m - mn) * mul);
        m = mn;
        // x = p * 2^11 = exp2(s * mul - (mn * mul - 11)), rounded to fp16:
        // one product per k-step (each weight moves by at most 2^-12 of
        // itself, independently of the others); l sums x and is scaled back
        // at the end
        float ps = 0.f;
        const float off = fmaf(mn, mul, -kPfPExp);
        pf_f16x4 phi[4];
#pragma unroll
        for (int i = 0; i < 16; i += 2) {  // pairs: one packed conversion each
            const float x0 = fast_exp2(fmaf(sv[i], mul, -off));
            const float x1 = fast_exp2(fmaf(sv[i + 1], mul, -off));
            const pf_f16x2 h = __builtin_convertvector((pf_f32x2){x0, x1}, pf_f16x2);
            ps += x0;
            ps += x1;
            phi[i >> 2][i & 3] = h[0];
            phi[i >> 2][(i & 3) + 1] = h[1];
        }
        lsum = fmaf(lsum, corr, ps);
        // accumulator rows 8*(i/4) + 4*hb + i%4 take the correction of their
        // own rows (held by lanes 0..31)
        if (__builtin_amdgcn_ballot_w64(corr != 1.f) != 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float ci = lane_read(corr, 8 * (i >> 2) + 4 * hb + (i & 3));
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) acc[nt][i] *= ci;
            }
        }
        if (t0 + 32 > t_end32) {  // the last sub-tile (wave-uniform)
            // zero the values of tokens past the last key (their weights are
            // zero, the stale halves need not be finite)
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const int n_ok = max(min(t_end32 - (t0 + 8 * kk + 4 * hb), 4), 0);
                const uint32_t mx_ = n_ok >= 2 ? 0xffffffffu : n_ok == 1 ? 0x0000ffffu : 0u;
                const uint32_t my_ = n_ok >= 4 ? 0xffffffffu : n_ok == 3 ? 0x0000ffffu : 0u;
#pragma unroll
                for (int nt = 0; nt < 4; ++nt) {
                    vop[kk][nt].x &= mx_;
                    vop[kk][nt].y &= my_;
                }
            }
        }
        // O[row][dim] += P[row][t] V[t][dim] on v_mfma_f32_32x32x16_f16: step
        // k2 takes tokens 16k2 .. 16k2+15, the lane's eight of them being
        // accumulator entries 8k2 .. 8k2+7 of the scores (tokens 16k2 + 4hb
        // + 0..3 and 16k2 + 8 + 4hb + 0..3); its B slice holds the values of
        // the same eight tokens (the two 8-token blocks' 4-token loads), so A
        // and B agree slot for slot
#pragma unroll
        for (int k2 = 0; k2 < 2; ++k2) {
            const pf_f16x8 ah = __builtin_shufflevector(phi[2 * k2], phi[2 * k2 + 1], 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int nt = 0; nt < 4; ++nt) {
                const pf_f16x8 b = __builtin_bit_cast(
                    pf_f16x8, make_uint4(vop[2 * k2][nt].x, vop[2 * k2][nt].y, vop[2 * k2 + 1][nt].x,
                                         vop[2 * k2 + 1][nt].y));
                acc[nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b, acc[nt], 0, 0, 0);
            }
        }
    };
    // sub-tiles in pairs with no exit between them (one register assignment
    // of the accumulators for the whole loop): an odd count ends with one
    // sub-tile past the last key, whose loads clamp to the last key's rows
    // and whose scores are all masked (weights and values zero)
    // (sub-tiles wholly below t_raw0 first, in pairs; the rest, the last
    // plain one of an odd count included, on the code that reads whole keys)
    const int n_plain = min(n_sub, t_raw0 / 32);
    int sub = 0;
    for (; sub + 1 < n_plain; sub += 2) {
        do_sub(std::false_type{}, ir_a, ir_b, sub);
        do_sub(std::false_type{}, ir_b, ir_a, sub + 1);
    }
    for (; sub < n_sub; sub += 2) {
        do_sub(std::true_type{}, ir_a, ir_b, sub);
        do_sub(std::true_type{}, ir_b, ir_a, sub + 1);
    }

    // 3. rows 8*(i/4) + 4*hb + i%4 of the accumulators: their l (the row's
    //    two lane halves summed), then the output
    const float L = lsum + lane_read(lsum, lane ^ 32);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int ri = 8 * (i >> 2) + 4 * hb + (i & 3);
        const float Li = lane_read(L, ri);
        const int rr = wv * 32 + ri;
        const int pp = rr / a.rep, hh = rr - pp * a.rep;
        const int64_t opos = (int64_t)pg * a.npos + pp;
        if (opos < a.t_q) {
            const int64_t off =
                ((bb * a.n_q_heads + (int64_t)kvh * a.rep + hh) * a.t_q + opos) * kPfD;
            const float inv = Li > 0.f ? 1.f / Li : 0.f;  // acc and l both carry 2^11
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                store_from_f32(a.out, a.out_dtype, off + 32 * nt + l32, acc[nt][i] * inv);
        }
    }
}

}  // namespace ss

using namespace ss;

// Query rows per workgroup of ss_prefill_attn_il8 (the rep of a GQA group
// must divide it) and the fewest query tokens it is meant for.
extern "C" int ss_prefill_rows_per_workgroup(void) { return kPfRows; }

static int prefill_impl(const void *q, int q_dtype, int64_t batch, int n_q_heads, int n_kv_heads,
                        int64_t t_q, int head_dim, float scale, const int32_t *perm,
                        const void *codebook, int n_blocks, int n_centroids, const uint8_t *idx,
                        int64_t cap, const void *values_il8, int v_dtype, int64_t cap_v,
                        int64_t t_kv, const void *kraw, const float *kfac, int64_t t_raw0,
                        int causal, int64_t q_offset, void *out, int out_dtype, void *stream) {
    SS_REQUIRE(q && codebook && idx && values_il8 && out, "null pointer argument");
    SS_REQUIRE(valid_dtype(q_dtype) && valid_dtype(out_dtype), "bad dtype code");
    SS_REQUIRE(batch >= 1 && n_q_heads >= 1 && n_kv_heads >= 1 && t_q >= 1 &&
                   n_q_heads % n_kv_heads == 0,
               "bad head/batch counts");
    SS_UNSUPPORTED(head_dim == kPfD && n_blocks == kPfNB,
                   "prefill kernel takes head_dim 128 with 16 blocks of 8 (got %d, %d)", head_dim,
                   n_blocks);
    SS_UNSUPPORTED(n_centroids >= 1 && n_centroids <= 256, "n_centroids %d unsupported (1..256)",
                   n_centroids);
    const int rep = n_q_heads / n_kv_heads;
    SS_UNSUPPORTED(kPfRows % rep == 0, "GQA group of %d query heads does not divide %d rows", rep,
                   kPfRows);
    SS_UNSUPPORTED(v_dtype == SS_F16, "interleaved values must be float16");
    SS_REQUIRE(cap_v % 8 == 0 && t_kv >= 0 && t_kv <= cap_v,
               "bad cap/t_kv (the value capacity a multiple of 8, t_kv <= it)");
    const bool raw = kraw != nullptr;
    SS_REQUIRE(!raw || (kfac && t_raw0 >= 0 && t_raw0 <= t_kv && t_raw0 <= cap),
               "whole keys need their factors and 0 <= t_raw0 <= min(t_kv, cap)");
    SS_REQUIRE(raw || t_kv <= cap, "t_kv exceeds the index capacity");
    SS_UNSUPPORTED(!raw || q_dtype != SS_F32,
                   "whole keys (a hybrid buffer) are taken with fp16 or bf16 queries only");
    SS_UNSUPPORTED(cap < (int64_t(1) << 24) && cap_v < (int64_t(1) << 24) &&
                       t_q + q_offset < (int64_t(1) << 30),
                   "prefill kernel takes caches below 2^24 tokens");
    SS_REQUIRE(q_offset >= 0, "negative q_offset");
    SS_REQUIRE(((uintptr_t)codebook % 16) == 0 && ((uintptr_t)idx % 16) == 0 &&
                   ((uintptr_t)values_il8 % 16) == 0,
               "codebook, idx and values must be 16-byte aligned");
    PrefillArgs a;
    a.q = q;
    a.q_dtype = q_dtype;
    a.n_q_heads = n_q_heads;
    a.n_kv_heads = n_kv_heads;
    a.rep = rep;
    a.t_q = t_q;
    a.scale = scale;
    a.perm = perm;
    a.codebook = static_cast<const uint4 *>(codebook);
    a.nct = (n_centroids + 15) / 16;
    a.cb_mul = reinterpret_cast<const float *>(static_cast<const char *>(codebook) +
                                               (size_t)(kPfNB / 4) * a.nct * 2 * kWave * 16);
    a.idx = idx;
    a.v8 = static_cast<const __half *>(values_il8);
    a.cap = cap;
    a.cap_v = cap_v;
    a.t_kv = t_kv;
    a.kraw = static_cast<const __half *>(kraw);
    a.kfac = kfac;
    a.t_raw0 = raw ? t_raw0 : t_kv;
    a.n_raw = raw ? t_kv - t_raw0 : 0;
    a.causal = causal ? 1 : 0;
    a.q_offset = q_offset;
    a.out = out;
    a.out_dtype = out_dtype;
    // fp16 and bf16 queries: waves of 32 rows on 32x32 products (each key
    // gather and value load serves twice the rows); fp32 queries, split into
    // fp16 hi and lo parts, keep 16-row waves (their second query operand
    // leaves no registers for 32 rows)
    const bool rows32 = q_dtype == SS_F16 || q_dtype == SS_BF16;
    a.npos = (rows32 ? kPfRows32 : kPfRows) / rep;
    const int64_t n_pg = (t_q + a.npos - 1) / a.npos;
    SS_UNSUPPORTED(n_pg <= 65535 && batch * n_kv_heads <= 0x7fffffff, "grid too large");
    a.n_pg = (int)n_pg;
    auto kern = rows32 ? prefill32_il8_kernel : prefill16_il8_kernel;
    static bool attr_set[2] = {false, false};
    if (!attr_set[rows32]) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kern),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 kPfLdsBytes);
        if (e != hipSuccess) return hip_fail(e, "hipFuncSetAttribute(prefill)");
        attr_set[rows32] = true;
    }
    hipLaunchKernelGGL(kern, dim3((unsigned)(batch * n_kv_heads), a.n_pg), dim3(kPfWaves * kWave),
                       kPfLdsBytes, reinterpret_cast<hipStream_t>(stream), a);
    SS_LAUNCH_CHECK("prefill_il8_kernel launch");
    return SS_OK;
}

extern "C" int ss_prefill_attn_il8(const void *q, int q_dtype, int64_t batch, int n_q_heads,
                                   int n_kv_heads, int64_t t_q, int head_dim, float scale,
                                   const int32_t *perm, const void *codebook, int n_blocks,
                                   int n_centroids, const uint8_t *idx, const void *values_il8,
                                   int v_dtype, int64_t cap, int64_t t_kv, int causal,
                                   int64_t q_offset, void *out, int out_dtype, void *stream) {
    return prefill_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                        codebook, n_blocks, n_centroids, idx, cap, values_il8, v_dtype, cap, t_kv,
                        nullptr, nullptr, 0, causal, q_offset, out, out_dtype, stream);
}

extern "C" int ss_prefill_attn_il8_hybrid(const void *q, int q_dtype, int64_t batch,
                                          int n_q_heads, int n_kv_heads, int64_t t_q,
                                          int head_dim, float scale, const int32_t *perm,
                                          const void *codebook, int n_blocks, int n_centroids,
                                          const uint8_t *idx, int64_t cap, const void *values_il8,
                                          int64_t cap_v, int64_t t_kv, const void *kraw,
                                          const float *kfac, int64_t t_raw0, int causal,
                                          int64_t q_offset, void *out, int out_dtype,
                                          void *stream) {
    SS_REQUIRE(kraw && kfac, "null pointer argument");
    SS_REQUIRE(((uintptr_t)kraw % 16) == 0, "kraw must be 16-byte aligned");
    return prefill_impl(q, q_dtype, batch, n_q_heads, n_kv_heads, t_q, head_dim, scale, perm,
                        codebook, n_blocks, n_centroids, idx, cap, values_il8, SS_F16, cap_v, t_kv,
                        kraw, kfac, t_raw0, causal, q_offset, out, out_dtype, stream);
}
