// Device helpers shared by the fused decode kernels (gfx950): bf16/f16
// packing, matrix-core wrappers, exact fp8 nibble conversion, 16-lane
// reductions and global-address-space loads.
#pragma once

#include "iq_common.h"

namespace {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
typedef __attribute__((ext_vector_type(4))) int i32x4;

template <bool F16>
__device__ __forceinline__ uint32_t pack2(float a, float b)
{
    if constexpr (F16) {
        f16x2 v = {(_Float16)a, (_Float16)b};
        return __builtin_bit_cast(uint32_t, v);
    } else {
        bf16x2 v = {(__bf16)a, (__bf16)b};
        return __builtin_bit_cast(uint32_t, v);
    }
}

template <bool F16>
__device__ __forceinline__ float to_f32(uint32_t h16)
{
    if constexpr (F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
    else return __uint_as_float(h16 << 16);
}

template <bool F16>
__device__ __forceinline__ float round_q(float v)
{
    return to_f32<F16>(pack2<F16>(v, 0.0f) & 0xffffu);
}

template <bool F16>
__device__ __forceinline__ f32x4 mma32(u32x4 a, u32x4 b, f32x4 c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
}

template <bool F16>
__device__ __forceinline__ f32x4 mma16(u32x2 a, u32x2 b, f32x4 c)
{
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                     0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b),
                                                        c, 0, 0, 0);
}

template <bool HI>
__device__ __forceinline__ f32x2 fp8x2(uint32_t bytes) { return __builtin_amdgcn_cvt_pk_f32_fp8(bytes, HI); }

// Reductions over the four 16-lane rows of a wavefront (lanes l, l ^ 16,
// l ^ 32, l ^ 48), result in every lane.  v_permlane16_swap with both operands
// equal to v yields rows (0, 0, 2, 2) and (1, 1, 3, 3); v_permlane32_swap
// yields the low and the high half.  No LDS traffic and no lane-index math.
__device__ __forceinline__ float xmax16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
}

__device__ __forceinline__ float xsum16(float v)
{
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

// Sum over the 16 lanes of each row, result in every lane of the row
// (DPP: swap neighbours, swap pairs, mirror the quads, mirror the halves).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float row_sum16(float v)
{
    v += dpp_f<0xb1>(v);     // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4e>(v);     // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);    // row_half_mirror
    return v + dpp_f<0x140>(v);   // row_mirror
}

// Loads through global-address-space pointers: the pointer table holds plain
// addresses, which would otherwise be dereferenced with flat instructions
// that every LDS wait must also drain.
template <class T>
__device__ __forceinline__ T ldg(const void *p)
{
    return *(const __attribute__((address_space(1))) T *)p;
}

__device__ __forceinline__ u32x4 ld16(const void *p) { return ldg<u32x4>(p); }

// base + a 32-bit byte offset: with `base` uniform this is the scalar-base
// form of the load (no 64-bit address arithmetic per lane)
template <class T>
__device__ __forceinline__ T ldg_at(const void *base, uint32_t off)
{
    return *(const __attribute__((address_space(1))) T *)((const char *)base + off);
}

template <class T>
__device__ __forceinline__ T ldnt_at(const void *base, uint32_t off)
{
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)((const char *)base + off));
}

// Streaming loads of packed payload, read once per call: the non-temporal hint
// keeps them from displacing small, re-read data (pointer tables, scales,
// queries, partials) in the caches.
template <class T>
__device__ __forceinline__ T ldnt(const void *p)
{
    return __builtin_nontemporal_load((const __attribute__((address_space(1))) T *)p);
}

// Orders LDS writes of this wavefront's lanes before reads of other lanes
// after it.  A wavefront's LDS operations complete in issue order, so no
// instruction is needed; the fence only keeps the compiler from reusing a
// value a lane read before (its per-thread model does not see other lanes'
// writes without synchronization).
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront"); }

constexpr float NEG_INF = -__builtin_inff();

// Partition partials in a workspace of rows * (128 + 2) floats: the
// unnormalized output rows first (rows x 128, 16-byte aligned), then the
// (max, sum) pairs (rows x 2), so that a merge reads whole 16-byte channel
// columns and the pairs of consecutive partitions from one cache line.
struct Partials {
    float *o;
    f32x2 *ml;
};

__device__ __forceinline__ Partials partials(float *ws, int64_t rows) { return {ws, (f32x2 *)(ws + rows * 128)}; }

// Workgroups go to the eight XCDs round-robin by linear id, and each XCD has
// its own L2.  For a 1-D grid of 64 * ceil(n / 8) workgroups this maps the
// linear id i to (item, slice) so that the eight slices of an item run on one
// XCD: a row the eight slices all read then misses one L2, not several.
// Items >= n are surplus workgroups that return at once.
__device__ __forceinline__ void iq_xcd_item_slice(int i, int &item, int &slice)
{
    const int r = i & 7, k = i >> 3;
    slice = k & 7;
    item = ((k >> 3) << 3) | r;
}

}  // namespace
