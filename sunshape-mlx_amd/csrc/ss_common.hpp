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

// Round a float32 to the precision of dtype dt (identity for float32).
__device__ __forceinline__ float round_to(int dt, float x) {
    if (dt == SS_F16) return __half2float(__float2half(x));
    if (dt == SS_BF16) return __bfloat162float(__float2bfloat16(x));
    return x;
}

__device__ __forceinline__ void store_from_f32(void *p, int dt, int64_t i, float x) {
    if (dt == SS_F32)
        reinterpret_cast<float *>(p)[i] = x;
    else if (dt == SS_F16)
        reinterpret_cast<__half *>(p)[i] = __float2half(x);
    else
        reinterpret_cast<__hip_bfloat16 *>(p)[i] = __float2bfloat16(x);
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

__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_mov<0xB1>(v));         // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp_mov<0x4E>(v));         // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp_mov<0x141>(v));        // row_half_mirror
    v = fmaxf(v, dpp_mov<0x140>(v));        // row_mirror
    v = fmaxf(v, dpp_mov<0x142, 0xa>(v));   // row_bcast:15 into rows 1, 3
    v = fmaxf(v, dpp_mov<0x143, 0xc>(v));   // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_mov<0xB1>(v);
    v += dpp_mov<0x4E>(v);
    v += dpp_mov<0x141>(v);
    v += dpp_mov<0x140>(v);
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
