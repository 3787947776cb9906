// Shared helpers for the SunShape HIP kernels (gfx950, wave64).
#pragma once

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sunshape_hip.h"

namespace ss {

// ---- host-side error reporting (thread-local text, see ss_last_error) ----
void set_error(const char *fmt, ...);
int hip_fail(hipError_t e, const char *what);
int device_cu_count();  // compute units of the current device (cached)

#define SS_REQUIRE(cond, ...)                                                   \
    do {                                                                        \
        if (!(cond)) {                                                          \
            ::ss::set_error(__VA_ARGS__);                                       \
            return SS_ERR_INVALID;                                              \
        }                                                                       \
    } while (0)

#define SS_UNSUPPORTED(cond, ...)                                               \
    do {                                                                        \
        if (!(cond)) {                                                          \
            ::ss::set_error(__VA_ARGS__);                                       \
            return SS_ERR_UNSUPPORTED;                                          \
        }                                                                       \
    } while (0)

#define SS_LAUNCH_CHECK(what)                                                   \
    do {                                                                        \
        hipError_t e_ = hipGetLastError();                                      \
        if (e_ != hipSuccess) return ::ss::hip_fail(e_, what);                  \
    } while (0)

inline bool valid_dtype(int dt) { return dt == SS_F32 || dt == SS_F16 || dt == SS_BF16; }
inline int dtype_bytes(int dt) { return dt == SS_F32 ? 4 : 2; }

// ---- device helpers ----
constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float load_as_f32(const void *p, int dt, int64_t i) {
    if (dt == SS_F32) return reinterpret_cast<const float *>(p)[i];
    if (dt == SS_F16) return __half2float(reinterpret_cast<const __half *>(p)[i]);
    return __bfloat162float(reinterpret_cast<const __hip_bfloat16 *>(p)[i]);
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(__half x) { return __half2float(x); }
__device__ __forceinline__ float to_f32(__hip_bfloat16 x) { return __bfloat162float(x); }

// Round a float32 to the precision of dtype dt (identity for float32).
__device__ __forceinline__ float round_to(int dt, float x) {
    if (dt == SS_F16) return __half2float(__float2half(x));
    if (dt == SS_BF16) return __bfloat162float(__float2bfloat16(x));
    return x;
}

// Value element j of token (b, h, t) -> the 8-token interleaved fp16 cache
// layout [b*n_h + h][cap/8][d][8] at position offset + t.
__device__ __forceinline__ void store_value_il8(__half *out, int64_t head, int64_t cap, int d,
                                                int64_t pos, int j, float x) {
    out[((head * (cap / 8) + pos / 8) * d + j) * 8 + (pos & 7)] = __float2half(x);
}

// Exponent s of the power of two 2^s that brings m = max |x| of a query row
// into [2^14, 2^15) as m * 2^-s, so every element of the row scaled by 2^-s
// lies within fp16's range and an element of at most 11 significant bits
// (fp16, bf16) stays exact unless it is below 2^-29 of m.  0 for a zero or
// non-finite m; clamped so both 2^s and 2^-s are normal floats.
__device__ __forceinline__ int row_exp_shift(float m) {
    if (!(m > 0.f) || !(m < INFINITY)) return 0;
    const int e = (int)((__float_as_uint(m) >> 23) & 0xffu) - 127;  // m in [2^e, 2^(e+1))
    return max(-126, min(126, e - 14));
}

// 2^s as a float for |s| <= 126.
__device__ __forceinline__ float exp2i(int s) { return __uint_as_float((uint32_t)(127 + s) << 23); }

__device__ __forceinline__ void store_from_f32(void *p, int dt, int64_t i, float x) {
    if (dt == SS_F32)
        reinterpret_cast<float *>(p)[i] = x;
    else if (dt == SS_F16)
        reinterpret_cast<__half *>(p)[i] = __float2half(x);
    else
        reinterpret_cast<__hip_bfloat16 *>(p)[i] = __float2bfloat16(x);
}

// Elements i .. i+3 of dtype dt: one 16-byte (float32) or 8-byte (16-bit)
// store when the destination is aligned for it, else four stores.
__device__ __forceinline__ void store4_from_f32(void *p, int dt, int64_t i, float x0, float x1, float x2,
                                                float x3) {
    if (dt == SS_F32) {
        float *q = reinterpret_cast<float *>(p) + i;
        if ((reinterpret_cast<uintptr_t>(q) & 15) == 0) {
            *reinterpret_cast<float4 *>(q) = make_float4(x0, x1, x2, x3);
            return;
        }
    } else {
        uint16_t *q = reinterpret_cast<uint16_t *>(p) + i;
        if ((reinterpret_cast<uintptr_t>(q) & 7) == 0) {
            auto bits = [&](float x) -> uint32_t {
                return dt == SS_F16 ? (uint32_t)__half_as_ushort(__float2half(x))
                                    : (uint32_t)__bfloat16_as_ushort(__float2bfloat16(x));
            };
            *reinterpret_cast<uint2 *>(q) = make_uint2(bits(x0) | (bits(x1) << 16), bits(x2) | (bits(x3) << 16));
            return;
        }
    }
    store_from_f32(p, dt, i, x0);
    store_from_f32(p, dt, i + 1, x1);
    store_from_f32(p, dt, i + 2, x2);
    store_from_f32(p, dt, i + 3, x3);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Wave64 reductions on DPP lane moves (no LDS round trips): butterflies inside
// each 16-lane row, then row_bcast:15 / row_bcast:31 fold the four rows into
// lane 63, which is read back as a wave-uniform value.
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float v) {
    const int x = __float_as_int(v);
    return __int_as_float(__builtin_amdgcn_update_dpp(x, x, CTRL, ROW_MASK, 0xf, false));
}

// Order-preserving map of a float onto a signed int (negative values have
// their magnitude bits flipped), so a float max can run as an integer max,
// which fuses with the DPP lane move (no NaN canonicalisation; NaN never
// occurs in the values reduced here).
__device__ __forceinline__ int ord_key(float f) {
    const int i = __float_as_int(f);
    return i ^ ((i >> 31) & 0x7fffffff);
}
__device__ __forceinline__ float ord_float(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7fffffff)); }

template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true);
}

__device__ __forceinline__ float wave_max_dpp(float v) {
    int k = ord_key(v);
    k = max(k, dpp_mov_i<0xB1>(k));   // quad_perm [1,0,3,2]
    k = max(k, dpp_mov_i<0x4E>(k));   // quad_perm [2,3,0,1]
    k = max(k, dpp_mov_i<0x141>(k));  // row_half_mirror
    k = max(k, dpp_mov_i<0x140>(k));  // row_mirror
    k = max(k, __builtin_amdgcn_update_dpp(k, k, 0x142, 0xa, 0xf, false));  // row_bcast:15 -> rows 1, 3
    k = max(k, __builtin_amdgcn_update_dpp(k, k, 0x143, 0xc, 0xf, false));  // row_bcast:31 -> rows 2, 3
    return ord_float(__builtin_amdgcn_readlane(k, 63));
}

// Four independent wave maxima, their butterfly steps interleaved so the
// DPP read-after-write waits of one chain are filled by the others.
__device__ __forceinline__ void wave_max4_dpp(const float (&v)[4], float (&out)[4]) {
    int k[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = ord_key(v[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], dpp_mov_i<0xB1>(k[i]));
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], dpp_mov_i<0x4E>(k[i]));
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], dpp_mov_i<0x141>(k[i]));
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], dpp_mov_i<0x140>(k[i]));
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], __builtin_amdgcn_update_dpp(k[i], k[i], 0x142, 0xa, 0xf, false));
#pragma unroll
    for (int i = 0; i < 4; ++i) k[i] = max(k[i], __builtin_amdgcn_update_dpp(k[i], k[i], 0x143, 0xc, 0xf, false));
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = ord_float(__builtin_amdgcn_readlane(k[i], 63));
}

// Four independent wave sums, steps interleaved (lane moves fused into the
// adds where the whole row is written).
__device__ __forceinline__ void wave_sum4_dpp(const float (&v)[4], float (&out)[4]) {
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = v[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] += __int_as_float(dpp_mov_i<0xB1>(__float_as_int(a[i])));
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] += __int_as_float(dpp_mov_i<0x4E>(__float_as_int(a[i])));
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] += __int_as_float(dpp_mov_i<0x141>(__float_as_int(a[i])));
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] += __int_as_float(dpp_mov_i<0x140>(__float_as_int(a[i])));
    // rows 1 and 3 add the total of the row before them, rows 0 and 2 add 0
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a[i] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[i]), 0x142, 0xa, 0xf, false));
#pragma unroll
    for (int i = 0; i < 4; ++i)
        a[i] += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a[i]), 0x143, 0xc, 0xf, false));
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(a[i]), 63));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += __int_as_float(dpp_mov_i<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp_mov_i<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp_mov_i<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp_mov_i<0x140>(__float_as_int(v)));
    // rows 1 and 3 add the total of the row before them; lanes of rows 0, 2
    // must not change, so they add 0
    {
        const int x = __float_as_int(v);
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false));
    }
    {
        const int x = __float_as_int(v);
        v += __int_as_float(__builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false));
    }
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Orders this wave's LDS accesses (all lanes) before the ones that follow:
// waits for outstanding LDS operations and stops the compiler from moving
// LDS accesses across the point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace ss
