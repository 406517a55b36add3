// Group-wise value-codec arithmetic for 16 consecutive 16-bit channels of
// one token (value_codec.py:57-71), shared by the row encoder and the page
// encoder so both produce the same bits.
//  * min / max use the NaN-propagating v_minimum3 / v_maximum3, so a NaN or
//    infinity anywhere in a group makes its offset or scale non-finite and
//    that single check replaces the per-value finiteness test;
//  * the quotient is clamped to [0, levels] before rounding (rint and an
//    integer clamp commute), so every value that can decide a code lies in
//    [0, levels] and the near-half test uses the fixed band 2^-16 >=
//    levels * 2^-20, with the IEEE division as the fallback;
//  * the codes are packed with exact fp32 multiply-adds (a sum of c * 4^e
//    stays below 2^16).
#pragma once

#include "iq_common.h"

typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;

// v of the lane selected by the DPP control CTRL (every lane active)
template <int CTRL>
__device__ __forceinline__ float grp_move(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// raw: 32 bytes = channels 16 j .. 16 j + 15 of one token; GL adjacent lanes
// form one group (every lane of the wavefront must call this together).
// Outputs the packed codes (BITS / 2 words, LSB-first), the group's f16
// offset and scale, and sets `bad` if a live token's parameters are not finite.
template <bool F16IN, int BITS, int GL>
__device__ __forceinline__ void v_encode16(const u32x4_t (&raw)[2], bool live, uint32_t (&word)[BITS / 2],
                                           uint16_t &off_h, uint16_t &sc_h, bool &bad)
{
    constexpr int L = (1 << BITS) - 1;
    float v[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const uint32_t w = raw[e >> 3][(e >> 1) & 3];
        const uint16_t hbits = (uint16_t)(e & 1 ? w >> 16 : w);
        v[e] = F16IN ? iq_f16_to_f32(hbits) : __uint_as_float(e & 1 ? w & 0xffff0000u : w << 16);
    }
    float lo = v[0], hi = v[0];
#pragma unroll
    for (int e = 1; e < 15; e += 2) {
        lo = __builtin_elementwise_minimum(__builtin_elementwise_minimum(lo, v[e]), v[e + 1]);
        hi = __builtin_elementwise_maximum(__builtin_elementwise_maximum(hi, v[e]), v[e + 1]);
    }
    lo = __builtin_elementwise_minimum(lo, v[15]);
    hi = __builtin_elementwise_maximum(hi, v[15]);
    // the group's GL lanes combine by DPP moves (no LDS round trip): lanes
    // i ^ 1 and i ^ 2 within a quad, then the mirrored half of the 8-lane
    // row, whose lanes lie in the other quad
    if constexpr (GL > 1) {
        lo = __builtin_elementwise_minimum(lo, grp_move<0xb1>(lo));      // quad_perm [1, 0, 3, 2]
        hi = __builtin_elementwise_maximum(hi, grp_move<0xb1>(hi));
    }
    if constexpr (GL > 2) {
        lo = __builtin_elementwise_minimum(lo, grp_move<0x4e>(lo));      // quad_perm [2, 3, 0, 1]
        hi = __builtin_elementwise_maximum(hi, grp_move<0x4e>(hi));
    }
    if constexpr (GL > 4) {
        lo = __builtin_elementwise_minimum(lo, grp_move<0x141>(lo));     // row_half_mirror
        hi = __builtin_elementwise_maximum(hi, grp_move<0x141>(hi));
    }
    static_assert(GL == 1 || GL == 2 || GL == 4 || GL == 8, "groups of 1, 2, 4 or 8 lanes");
    off_h = iq_f32_to_f16(lo);
    float s = __fsub_rn(hi, lo) / (float)L;
    s = s < 6.103515625e-05f ? 6.103515625e-05f : s;
    sc_h = iq_f32_to_f16(s);
    const float off = iq_f16_to_f32(off_h), sc = iq_f16_to_f32(sc_h);
    bad |= live && !(iq_isfinite(off) && iq_isfinite(sc));

    const float rsc = __builtin_amdgcn_rcpf(sc);
    float q[16], dev = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) {
        const float c = __builtin_amdgcn_fmed3f(__fmul_rn(__fsub_rn(v[e], off), rsc), 0.0f, (float)L);
        q[e] = __builtin_rintf(c);
        dev = fmaxf(dev, fabsf(__fsub_rn(q[e], c)));
    }
    if (dev >= 0.5f - 0x1p-16f) {     // a quotient near a half-integer: the IEEE division decides
#pragma unroll
        for (int e = 0; e < 16; ++e)
            q[e] = fminf(fmaxf(rintf(__fsub_rn(v[e], off) / sc), 0.0f), (float)L);
    }
    if constexpr (BITS == 2) {
        float p0 = q[0], p1 = q[8];
#pragma unroll
        for (int e = 1; e < 8; ++e) {
            p0 = __builtin_fmaf(q[e], (float)(1 << (2 * e)), p0);
            p1 = __builtin_fmaf(q[8 + e], (float)(1 << (2 * e)), p1);
        }
        word[0] = (uint32_t)p0 | ((uint32_t)p1 << 16);
    } else {
        uint32_t w[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float p = q[4 * g];
#pragma unroll
            for (int e = 1; e < 4; ++e) p = __builtin_fmaf(q[4 * g + e], (float)(1 << (4 * e)), p);
            w[g] = (uint32_t)p;
        }
        word[0] = w[0] | (w[1] << 16);
        word[BITS / 2 - 1] = w[2] | (w[3] << 16);
    }
}
