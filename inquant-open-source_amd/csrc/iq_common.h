// Shared device/host helpers for the InQuant HIP library (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/inquant_hip.h"

// ---------------------------------------------------------------- errors

// Records a message for iq_last_error() and returns the status code.
int iq_fail(int status, const char *fmt, ...);

#define IQ_CHECK_ARG(cond, ...)                                   \
    do {                                                          \
        if (!(cond)) return iq_fail(IQ_ERR_ARG, __VA_ARGS__);     \
    } while (0)

#define IQ_CHECK_LAUNCH(what)                                                         \
    do {                                                                              \
        hipError_t e_ = hipGetLastError();                                            \
        if (e_ != hipSuccess) return iq_fail(IQ_ERR_DEVICE, "%s launch: %s", what,    \
                                             hipGetErrorString(e_));                  \
    } while (0)

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float iq_bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t iq_f32_to_bf16(float f)
{
    // gfx950 lowers this to v_cvt_pk_bf16_f32 (round to nearest even).
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float iq_f16_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

__device__ __forceinline__ uint16_t iq_f32_to_f16(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Load element i of a tensor of dtype `dt` as fp32 (exact for bf16/f16/f32).
__device__ __forceinline__ float iq_load_f32(const void *p, int64_t i, int dt)
{
    switch (dt) {
    case IQ_BF16: return iq_bf16_to_f32(((const uint16_t *)p)[i]);
    case IQ_F16: return iq_f16_to_f32(((const uint16_t *)p)[i]);
    case IQ_F64: return (float)((const double *)p)[i];
    default: return ((const float *)p)[i];
    }
}

// Round an fp32 value to the nearest value of dtype `dt` (fp32 result).
__device__ __forceinline__ float iq_round_to(float v, int dt)
{
    if (dt == IQ_BF16) return iq_bf16_to_f32(iq_f32_to_bf16(v));
    if (dt == IQ_F16) return iq_f16_to_f32(iq_f32_to_f16(v));
    return v;
}

__device__ __forceinline__ void iq_store_as(void *p, int64_t i, float v, int dt)
{
    switch (dt) {
    case IQ_BF16: ((uint16_t *)p)[i] = iq_f32_to_bf16(v); break;
    case IQ_F16: ((uint16_t *)p)[i] = iq_f32_to_f16(v); break;
    case IQ_F64: ((double *)p)[i] = (double)v; break;
    default: ((float *)p)[i] = v; break;
    }
}

// rint(RN(a / b)) for normal b, given rcp_b = v_rcp_f32(b) (within 1 ulp of
// 1 / b): the reciprocal product q is within 2^-21 |q|
// of the quotient, so its rounding equals that of the IEEE quotient unless q
// lies within 2^-20 |q| of a half-integer, where the IEEE division decides.
__device__ __forceinline__ float iq_rint_div(float a, float b, float rcp_b)
{
    const float q = __fmul_rn(a, rcp_b);
    const float r = rintf(q);
    const float d = 0.5f - fabsf(__fsub_rn(q, r));
    if (d > fabsf(q) * 0x1p-20f) return r;
    return rintf(a / b);
}

__device__ __forceinline__ bool iq_isfinite(float x) { return (__float_as_uint(x) & 0x7f800000u) != 0x7f800000u; }

// ---------------------------------------------------------------- direct loads

// One 16-byte-per-lane direct global -> LDS load: lane l's 16 bytes at
// base + voff land at LDS byte lds_base + 16 l (base and lds_base
// wave-uniform).  Issued from inline assembly so that the compiler does not
// treat every later LDS read as possibly dependent on it (it would wait for
// all loads in flight); callers wait explicitly (s_waitcnt vmcnt, then a
// barrier).  The assembly sets M0 itself; nothing the compiler generates for
// the kernels that use it reads M0 (M0 is a reserved register, so it cannot
// be listed as clobbered).
__device__ __forceinline__ void lds_load16(const void *base, uint32_t voff, uint32_t lds_base)
{
    // the operands are wave-uniform: make them scalar registers explicitly
    // (readfirstlane returns int: widen through uint32_t, not by sign extension)
    const uint64_t b = (uint64_t)(uintptr_t)base;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)b);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(b >> 32));
    const uint64_t sb = (uint64_t)lo | ((uint64_t)hi << 32);
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sb),
                 "s"(__builtin_amdgcn_readfirstlane(lds_base))
                 : "memory");
}

// ---------------------------------------------------------------- torch CPU reduction orders

// Columns [0, iq_cascade_columns(D)) of an outer reduction are summed by
// torch's cascade; the rest by its interleaved row_sum (8-float vectors).
__host__ __device__ __forceinline__ int64_t iq_cascade_columns(int64_t D)
{
    return D >= 8 ? (D / 32) * 32 : (D / 4) * 4;
}

__device__ __forceinline__ int iq_ceil_log2(int64_t x)
{
    int r = 0;
    if (x <= 1) return 0;
    x -= 1;
    while (x) { ++r; x >>= 1; }
    return r;
}

// Incremental form of torch's 4-level cascade sum (aten multi_row_sum).
struct IqCascade {
    float acc[4];
    int64_t i;      // values consumed
    int lp;         // log2 of the chunk length
    __device__ void init(int64_t n)
    {
        acc[0] = acc[1] = acc[2] = acc[3] = 0.0f;
        i = 0;
        lp = iq_ceil_log2(n) / 4;
        if (lp < 4) lp = 4;
        full = (n >> lp) << lp;   // values that belong to complete chunks
    }
    int64_t full;
    __device__ void add(float x)
    {
        acc[0] = __fadd_rn(acc[0], x);
        ++i;
        if (i <= full && (i & (((int64_t)1 << lp) - 1)) == 0) {
            const int64_t mask = ((int64_t)1 << lp) - 1;
            for (int j = 1; j < 4; ++j) {
                acc[j] = __fadd_rn(acc[j], acc[j - 1]);
                acc[j - 1] = 0.0f;
                if ((i & (mask << (j * lp))) != 0) break;
            }
        }
    }
    __device__ float finish() const
    {
        float s = acc[0];
        s = __fadd_rn(s, acc[1]);
        s = __fadd_rn(s, acc[2]);
        s = __fadd_rn(s, acc[3]);
        return s;
    }
};
