// Exact block-VQ encode by one wave, shared by the encoder (encode.hip) and
// the decode step that appends its new tokens in the same launch
// (decode.hip).  A block's index is the nearest centroid in squared L2
// (reference kernels.py:995-1027, ties to the lowest index), ranked in
// float32 and re-ranked in float64 when the runner-up is within kSuspectRel
// of the best (wider than the float32 error of an 8-term sum of squares).
#pragma once

#include "ss_common.hpp"

namespace ss {

constexpr float kSuspectRel = 4e-6f;

// Exact nearest codeword of one block, the whole wave cooperating: lanes
// split the codebook, direct-form float32 ranking, (distance, index)
// reduced across the wave with lowest-index ties, and a float64 re-rank
// when the runner-up is within kSuspectRel of the best.
template <int BD>
__device__ __forceinline__ int exact_block_wave(const float (&kv)[BD], const float *cb, int nc, int lane) {
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
    return bi == 0x7fffffff ? 0 : bi;  // every distance NaN: the reference keeps index 0
}

// The lane's centroids c = lane + 64 i (i < 4; clamped to the last one) of
// an 8-dim block's codebook cbb [nc][8], nc <= 256.
__device__ __forceinline__ void load_centroids8(const float *cbb, int nc, int lane, float4 (&cv)[4][2]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = min(lane + kWave * i, nc - 1);
        cv[i][0] = *reinterpret_cast<const float4 *>(cbb + c * 8);
        cv[i][1] = *reinterpret_cast<const float4 *>(cbb + c * 8 + 4);
    }
}

// Dims blk*8 .. blk*8+7 of a key in the codec's basis (dim j from key dim
// perm[j], perm null = identity), from a key row held as kr[u] = dim
// lane + 64u (dims < 256): every lane gets all eight, by shuffles.
__device__ __forceinline__ void block_dims8(const float (&kr)[4], const int32_t *perm, int blk,
                                            float (&kv)[8]) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int j = blk * 8 + k;
        const int src = __builtin_amdgcn_readfirstlane(perm ? perm[j] : j);  // wave-uniform
        const int u = (src >> 6) & 3;
        const float x = u == 0 ? kr[0] : u == 1 ? kr[1] : u == 2 ? kr[2] : kr[3];
        kv[k] = __shfl(x, src & (kWave - 1));
    }
}

// exact_block_wave for 8-dim blocks of at most 256 centroids with the
// lane's centroids (c = lane + 64 i) already in registers, so their loads
// overlap the key's; the same float steps, ties and refinement.
__device__ __forceinline__ int exact_block_wave_regs8(const float (&kv)[8], const float4 (&cv)[4][2],
                                      const float *cb, int nc, int lane) {
    float best = INFINITY, second = INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = lane + kWave * i;
        if (c < nc) {
            const float x[8] = {cv[i][0].x, cv[i][0].y, cv[i][0].z, cv[i][0].w,
                                cv[i][1].x, cv[i][1].y, cv[i][1].z, cv[i][1].w};
            float df = kv[0] - x[0];
            float d = df * df;
#pragma unroll
            for (int k = 1; k < 8; ++k) {
                df = kv[k] - x[k];
                d = fmaf(df, df, d);
            }
            const bool lt = d < best;
            second = lt ? best : fminf(second, d);
            bi = lt ? c : bi;
            best = lt ? d : best;
        }
    }
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
            for (int k = 0; k < 8; ++k) {
                const double df = (double)kv[k] - (double)cb[c * 8 + k];
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
    return bi == 0x7fffffff ? 0 : bi;
}

}  // namespace ss
